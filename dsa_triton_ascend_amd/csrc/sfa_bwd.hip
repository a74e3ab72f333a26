// Sparse flash attention backward (MLA-absorb, N2 = 1) for gfx950.
//
// Semantics: sparse_flash_attention_grad_numpy.py:34-143 (the golden), the
// inputs and outputs of sparse_flash_attention_grad_triton.py:498-677. Per
// query row and head, with the forward's output O and softmax stats:
//   P  = exp(score - sm_max) / sm_sum,  score = (q . k + q_rope . k_rope) * scale
//   dS = P * (dO . k_nope - dO . O) * scale
//   d_query | d_query_rope = dS @ [k_nope | k_rope]          (per row)
//   d_key | d_key_rope    += dS^T @ [q_nope | q_rope]        (scatter over tokens)
//   d_value               += P^T @ dO                        (scatter over tokens)
//
// d_key / d_value are computed as dense GEMMs instead of per-(row, token)
// scatters: per batch, the P and dS of every (query row, head, key token) go to
// two token-major buffers PT[token][row * N1 + head] (zero where a row does not
// select the token), and then
//   [d_key | d_key_rope][t, :] = sum_k dS_T[t, k] [q | q_rope][k, :]
//   d_value[t, :]             = sum_k P_T[t, k]  d_out[k, :]
// with k running over the batch's (row, head) pairs. At the reference's shapes a
// key token is selected by a large share of the rows (half of them at
// S2 = 2 * topK), so these dense products cost less than scattering
// (D + Dr + D) fp32 atomics per selected (row, token, head block).
//
// Launches:
//  1. the forward's token-list kernels (the golden's gather order, physical key
//     rows), so both passes select exactly the same tokens;
//  2. sfa_bwd_geo_kernel -- per-batch offsets of the dense buffers; clears the
//     fp32 accumulators and the used part of the dense buffers;
//  3. sfa_bwd_rows_kernel -- one work-group (8 waves, two per SIMD) per (query
//     row, block of 32 heads). Q | Q rope and dO of the block sit in LDS for the
//     whole row; the row's tokens are processed in tiles of 32 gathered [D | Dr] rows:
//       * S^T = K Q^T and dP^T = K_nope dO^T on v_mfma_f32_32x32x16 (tokens as
//         M, heads as N), their k-ranges split in quarters over waves 0-3 (S^T)
//         and 4-7 (dP^T) and summed through LDS;
//       * P and dS in fp32, stored in the io dtype to the dense buffers (32
//         consecutive heads of one token per store group) and dS also to LDS as
//         [head][token];
//       * dQ[head, col] += dS K, each wave owning an eighth of the 32-column
//         blocks, the K operand read with ds_read_b64_tr_b16 from the tile;
//  4. two library GEMMs per batch (hipBLASLt, loaded on first use; a fixed algorithm per
//     shape, so results are reproducible across processes; bf16/fp16 in and out, fp32
//     accumulation): [d_key | d_key_rope] = dS_T [q | q_rope] (one product: the rows
//     kernel writes [q | q_rope] to a concatenated workspace buffer as it loads it;
//     a separate 64-column d_key_rope product took 0.10 ms) and d_value = P_T d_out,
//     into a batch-contiguous staging area of the workspace, each as one
//     strided-batched product over BSPLIT chunks of the contraction with fp32
//     partials (the outputs alone have too few tiles to fill the GPU); these are
//     plain dense products, the kind of work a tuned library GEMM does best
//     (measured 0.35 ms at the grad perf shape against 0.74 ms for the hand-written
//     GEMM kernels they replaced);
//  5. sfa_bwd_place_kernel -- adds each batch's staged partials into key rows
//     key_start[b] + t (io dtype) and writes zeros to the key rows no batch covers.
#include <dlfcn.h>

#include <climits>
#include <type_traits>
#include <map>
#include <mutex>
#include <string>
#include <tuple>

#include <hipblaslt/hipblaslt.h>   // types and prototypes only: the library is loaded with dlopen

#include "dsa_common.hpp"

namespace dsa {
namespace {

constexpr int BDR = 64;     // rope width
constexpr int BH = 32;      // heads per work-group (rows kernel)
constexpr int BT = 32;      // tokens per tile
constexpr int BWV = 8;      // waves per work-group (two per SIMD)
constexpr float BLOG2E = 1.4426950408889634f;
constexpr int GBK = 64;     // dense rows are padded to a multiple of 64 (row, head) pairs
constexpr size_t LT_WS = (size_t)128 << 20;  // workspace offered to the library GEMMs
constexpr int LT_CANDIDATES = 64;            // length of the heuristic's ranked list
// Split of the products' contraction (the batch's (row, head) pairs): with M = key rows
// and N = D + Dr or D the output has few tiles (about 64 - 144 at the grad perf shape for
// 256 CUs), so the contraction is cut into BSPLIT chunks, run as one strided-batched
// GEMM writing fp32 partials that the place kernel adds.
constexpr int BSPLIT = 4;

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

template <int D> struct BCfg {
  static constexpr int DT = D + BDR;                   // [nope | rope] width
  static constexpr int QP = DT + 8;                    // Q / K row pitch: odd count of 16-byte units
  static constexpr int OP = D + 8;                     // dO row pitch
  static constexpr int PP = BT + 8;                    // dS row pitch
  static constexpr int NBQ = DT / 32;                  // 32-column blocks of dQ
  static constexpr int JQ = (NBQ + BWV - 1) / BWV;     // dQ blocks per wave, at most
  static constexpr int KS_S = DT / 16;                 // k-steps of S^T
  static constexpr int KS_P = D / 16;                  // of dP^T
  static_assert(KS_S % 4 == 0 && KS_P % 4 == 0, "k-ranges split in quarters");
  static constexpr int KCH = (BT * (DT / 8) + BWV * 64 - 1) / (BWV * 64);   // 16-byte gather chunks per thread
  // words of the selected-token bitmap (batches of up to 32 ZBW key tokens clear their
  // dense slices in the rows kernel); D = 128 keeps two work-groups per CU
  static constexpr int ZBW = D == 128 ? 2048 : 4096;
};

// MFMA 32x32x16 operand whose K runs down the rows of a row-major 16-bit LDS
// array X (pitch in elements): lane l receives X[k0 + 8 (l / 32) + j][c0 + l % 32],
// j = 0..7, from two transposed 8-byte reads (rows k and k + 4 of its group).
__device__ __forceinline__ uint4 tr_frag(const uint16_t* X, int pitch, int c0, int k0, int lane) {
  const int g16 = lane >> 4, c16 = lane & 15;
  const int col = c0 + (g16 & 1) * 16 + 4 * (c16 & 3);
  const int k = k0 + (g16 >> 1) * 8 + (c16 >> 2);
  const uint2 lo = ds_read_tr(X + k * pitch + col);
  const uint2 hi = ds_read_tr(X + (k + 4) * pitch + col);
  return make_uint4(lo.x, lo.y, hi.x, hi.y);
}

struct BwdWs {
  int64_t* boff;   // [batch + 1] dense-buffer offsets (elements)
  int64_t* boffk;  // [batch + 1] staged-row offsets (prefix of nk)
  float* skc;      // staged [split][sum nk, D + Dr] d_key | d_key_rope partials (fp32)
  uint16_t* qcat;  // [total_rows * N1, D + Dr] q | q_rope (written by the rows kernel)
  uint16_t* gocat; // [total_rows * N1, D] d_out (written by the rows kernel)
  float* sv;       // staged [split][sum nk, D] d_value partials (fp32)
  int split;       // partials per staged row (1 or BSPLIT)
  void* lt_ws;     // LT_WS bytes for the library GEMMs
  uint16_t* dst;   // dS_T dense buffer (io dtype)
  uint16_t* pt;    // P_T dense buffer (io dtype)
  int64_t cap;     // elements per dense buffer
  int zfuse;       // the rows kernel writes the zeros of the dense buffers (no clear kernels)
};

// Dense geometry of batch b: query rows [rs, rs + nq), key rows [ks, ks + nk)
// (the tokens a row of the batch can select, t < min(act_k, S2)), dense rows of
// kp = nq * N1 rounded up to GBK elements. The host computes the same nk and kp from
// its copies of row_start / act_k (bwd_host_geo) to size and address the GEMMs.
struct BatchGeo {
  int rs, nq, ks, nk, kp;
};

__host__ __device__ inline int batch_nk(int act_k, int s2) { return act_k < 0 ? 0 : (act_k < s2 ? act_k : s2); }

__host__ __device__ inline int dense_row(int nq, int n1) { return (nq * n1 + GBK - 1) / GBK * GBK; }

__device__ __forceinline__ BatchGeo batch_geo(const SfaArgs& f, int b) {
  BatchGeo g;
  g.rs = f.row_start[b];
  g.nq = f.row_start[b + 1] - g.rs;
  g.ks = f.key_start[b];
  g.nk = batch_nk(f.act_k[b], f.s2);
  g.kp = dense_row(g.nq, f.n1);
  return g;
}

// One work-group: per-batch offsets of the dense buffers (prefix of nk * kp).
__global__ __launch_bounds__(256) void sfa_bwd_geo_kernel(SfaArgs f, BwdWs w) {
  __shared__ int64_t part[256];
  const int tid = threadIdx.x;
  const int per = (f.batch + 255) / 256;
  const int b0 = tid * per;
  int64_t sum = 0;
  for (int b = b0; b < b0 + per && b < f.batch; ++b) {
    const BatchGeo g = batch_geo(f, b);
    sum += (int64_t)g.nk * g.kp;
  }
  part[tid] = sum;
  __syncthreads();
  if (tid == 0) {
    int64_t run = 0;
    for (int i = 0; i < 256; ++i) {
      const int64_t v = part[i];
      part[i] = run;
      run += v;
    }
  }
  __syncthreads();
  int64_t off = part[tid];
  for (int b = b0; b < b0 + per && b < f.batch; ++b) {
    w.boff[b] = off;
    const BatchGeo g = batch_geo(f, b);
    off += (int64_t)g.nk * g.kp;
  }
  if (tid == 255) w.boff[f.batch] = off;
  // staged-row offsets: the same prefix over nk
  __syncthreads();
  int64_t sk = 0;
  for (int b = b0; b < b0 + per && b < f.batch; ++b) sk += batch_nk(f.act_k[b], f.s2);
  part[tid] = sk;
  __syncthreads();
  if (tid == 0) {
    int64_t run = 0;
    for (int i = 0; i < 256; ++i) {
      const int64_t v = part[i];
      part[i] = run;
      run += v;
    }
  }
  __syncthreads();
  off = part[tid];
  for (int b = b0; b < b0 + per && b < f.batch; ++b) {
    w.boffk[b] = off;
    off += batch_nk(f.act_k[b], f.s2);
  }
  if (tid == 255) w.boffk[f.batch] = off;
}

// Clears n4 16-byte words of p (accumulators); dense buffers: up to the used size
__global__ void sfa_bwd_zero_kernel(uint4* p, int64_t n4, const int64_t* used_elems, int64_t cap_elems) {
  if (used_elems) {
    const int64_t u = *used_elems < cap_elems ? *used_elems : cap_elems;
    const int64_t n8 = (u + 7) / 8;
    n4 = n8 < n4 ? n8 : n4;
  }
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = make_uint4(0, 0, 0, 0);
}

template <int IO, int D>
__global__ __launch_bounds__(BWV * 64) void sfa_bwd_rows_kernel(SfaBwdArgs a, SfaTokenLists tl, BwdWs w) {
  using C = BCfg<D>;
  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][BT * C::QP];    // [token][nope | rope], tiles t, t - 1
  __shared__ __attribute__((aligned(16))) uint16_t dSs[2][BH * C::PP];   // [head][token], tiles t, t - 1
  __shared__ float part[BWV][16][64];   // S^T (waves 0-3) / dP^T (4-7) k-range partials, MFMA layout
  __shared__ int s_tok[2][BT];          // the tile's token index within the batch (-1: none)
  __shared__ int s_idr[4][BT];          // token-id ring: the ids of tile t in slot t % 4
  __shared__ float s_m[BH], s_il[BH], s_dl[BH];
  __shared__ uint32_t s_sel[C::ZBW];    // the batch tokens this row writes to the dense buffers

  const SfaArgs& f = a.f;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = f.total_rows - 1 - (int)blockIdx.x;   // long (late causal) rows first
  const int n1 = f.n1;
  const int h0 = blockIdx.y * BH;
  const int hn = n1 - h0 < BH ? n1 - h0 : BH;          // heads of this block
  const int krows = f.key_rows < INT_MAX ? (int)f.key_rows : INT_MAX;
  const int ntok = tl.counts[r];
  const int32_t* toks = tl.tokens + (int64_t)r * tl.tstride;
  const uint16_t* kb = reinterpret_cast<const uint16_t*>(f.k);
  const uint16_t* krb = reinterpret_cast<const uint16_t*>(f.kr);
  const uint4 z4 = make_uint4(0, 0, 0, 0);
  // dense-buffer row base of this (row, head block): token t of the batch at
  // dbase + t * kp; writes only when the batch's block fits the buffers
  const int b = batch_of_row(f.row_start, f.batch, r);
  const BatchGeo g = batch_geo(f, b);
  const int rl = r - g.rs;
  const bool dense_ok = rl >= 0 && rl < g.nq && w.boff[b + 1] <= w.cap;
  const int64_t dbase = w.boff[b] + (int64_t)rl * n1 + h0;
  const bool zf = w.zfuse && dense_ok;   // the host checked nk <= 32 ZBW and N1 % 8 == 0

  // ---- the block's Q | Q rope and dO (rows past the heads are zero), stats
  {
    const uint16_t* qb = reinterpret_cast<const uint16_t*>(f.q);
    const uint16_t* qrb = reinterpret_cast<const uint16_t*>(f.qr);
    const uint16_t* gob = reinterpret_cast<const uint16_t*>(a.d_out);
    for (int i = tid; i < BH * (C::DT / 8); i += BWV * 64) {
      const int h = i / (C::DT / 8), c = (i % (C::DT / 8)) * 8;
      if (h < hn) {
        const int64_t hr = (int64_t)r * n1 + h0 + h;
        const uint4 v = c < D ? ldg16(qb + hr * D + c) : ldg16(qrb + hr * BDR + (c - D));
        // the B operand of the [d_key | d_key_rope] product; zeros for a row without tokens
        // (inactive rows among them), so that whatever its q holds (NaN included) never
        // reaches d_key through the zero columns of its dS
        stg16(w.qcat + hr * C::DT + c, ntok > 0 ? v : z4);
      }
    }
    // delta = dO . O (fp32) per head: 8 threads per head, D/8 columns each
    const uint16_t* ob = reinterpret_cast<const uint16_t*>(a.out);
    const int h = tid >> 3, part8 = tid & 7;
    float dl = 0.f;
    if (h < hn) {
      const int64_t hr = (int64_t)r * n1 + h0 + h;
      for (int c = part8 * 8; c < D; c += 64) {
        const uint4 o = ldg16(ob + hr * D + c), gv = ldg16(gob + hr * D + c);
        // the B operand of the d_value product (zeros for a row without tokens, as above)
        stg16(w.gocat + hr * D + c, ntok > 0 ? gv : z4);
        const uint32_t ow[4] = {o.x, o.y, o.z, o.w}, gw[4] = {gv.x, gv.y, gv.z, gv.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          dl += to_f32<IO>((uint16_t)(ow[j] & 0xFFFFu)) * to_f32<IO>((uint16_t)(gw[j] & 0xFFFFu));
          dl += to_f32<IO>((uint16_t)(ow[j] >> 16)) * to_f32<IO>((uint16_t)(gw[j] >> 16));
        }
      }
    }
    dl += __shfl_xor(dl, 1);
    dl += __shfl_xor(dl, 2);
    dl += __shfl_xor(dl, 4);
    if (part8 == 0 && h < BH) {
      float m = 0.f, il = 0.f;
      if (h < hn) {
        const int64_t hr = (int64_t)r * n1 + h0 + h;
        m = a.sm_max[hr];
        const float l = a.sm_sum[hr];
        il = l > 0.f ? 1.f / l : 0.f;
      }
      s_m[h] = m * BLOG2E;
      s_il[h] = il;
      s_dl[h] = h < hn ? dl : 0.f;
    }
  }

  f32x16 dq[C::JQ];
#pragma unroll
  for (int jj = 0; jj < C::JQ; ++jj)
#pragma unroll
    for (int i = 0; i < 16; ++i) dq[jj][i] = 0.f;
  const float sl2 = f.scale * BLOG2E;
  // the B operand of this wave's S^T / dP^T quarter (Q | Q rope or dO of head h0 + lane % 32,
  // the same for every tile) stays in VGPRs, loaded once from global memory
  constexpr int NBQ4 = C::KS_S / 4;   // k-steps of an S^T quarter (>= those of a dP^T quarter)
  uint4 bq[NBQ4];
  {
    const int hb = lane & 31;
    const int64_t hr = (int64_t)r * n1 + h0 + (hb < hn ? hb : 0);
    if (wave < 4) {
      const uint16_t* qb = reinterpret_cast<const uint16_t*>(f.q);
      const uint16_t* qrb = reinterpret_cast<const uint16_t*>(f.qr);
#pragma unroll
      for (int i = 0; i < NBQ4; ++i) {
        const int c = ((wave & 3) * (C::KS_S / 4) + i) * 16 + (lane >> 5) * 8;
        bq[i] = ldg16_or0(hb < hn, c < D ? qb + hr * D + c : qrb + hr * BDR + (c - D));
      }
    } else {
      const uint16_t* gob = reinterpret_cast<const uint16_t*>(a.d_out);
#pragma unroll
      for (int i = 0; i < NBQ4; ++i) {
        const int c = ((wave & 3) * (C::KS_P / 4) + i) * 16 + (lane >> 5) * 8;
        bq[i] = ldg16_or0(hb < hn && i < C::KS_P / 4, gob + hr * D + (i < C::KS_P / 4 ? c : 0));
      }
    }
  }

  // ---- gathers of a tile's [nope | rope] rows into registers (rows outside the key
  // tensors and slots past the list are zero), two register sets: the next two
  // tiles' rows are in flight while one is computed
  constexpr int KCH = C::KCH;   // 16-byte chunks per thread (the last one on part of the threads)
  constexpr int NCH = BT * (C::DT / 8);
  uint4 ka[KCH], kbr[KCH];
  int pa = -1, pb = -1;
  auto gather = [&](int t0, uint4 (&kreg)[KCH], int& ptok) __attribute__((always_inline)) {
    const int nvt = ntok - t0 < BT ? ntok - t0 : BT;
    const int* ids = s_idr[(t0 / BT) & 3];
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int idx = tid + BWV * 64 * i;
      const int t = idx / (C::DT / 8), c = (idx % (C::DT / 8)) * 8;
      const int p = idx < NCH && t < nvt ? ids[t] : -1;
      uint4 v = z4;
      if ((uint32_t)p < (uint32_t)krows)
        v = c < D ? ldg16(kb + (int64_t)p * D + c) : ldg16(krb + (int64_t)p * BDR + (c - D));
      kreg[i] = v;
    }
    if (tid < BT) {
      const int p = tid < nvt ? ids[tid] : -1;
      const int tb = p - g.ks;   // token index within the batch
      ptok = dense_ok && (uint32_t)p < (uint32_t)krows && tb >= 0 && tb < g.nk ? tb : -1;
    }
  };
  // The token ids reach the gathers through the LDS ring s_idr: threads < 32 load
  // the ids of tile t+4 during tile t (before that tile's row loads, so waiting
  // for them never waits for rows) and publish them at the start of tile t+1;
  // the rows of tile t+2 are gathered during tile t from the ids published at
  // tile t-1. No gather waits on a global id load.
  int idreg = -1;
  auto load_ids = [&](int t0) __attribute__((always_inline)) {
    if (tid < BT) idreg = t0 + tid < ntok ? toks[t0 + tid] : -1;
  };
  // one tile: its rows from the register set `kreg` to LDS, then that set is
  // refilled with the rows two tiles ahead. Barriers order LDS only (lds_barrier):
  // a full __syncthreads() would also wait for the gathers in flight.
  // ---- dQ[head, col] += dS[head, token] K[token, col] of tile tp (this wave's column
  // blocks; every operand of the phase is requested before its MFMAs)
  auto dq_phase = [&](int tp) __attribute__((always_inline)) {
    const uint16_t* const kt = Ks[tp & 1];
    const uint16_t* const dst = dSs[tp & 1];
    uint4 av[BT / 16], bv[C::JQ][BT / 16];
#pragma unroll
    for (int kq = 0; kq < BT / 16; ++kq)
      av[kq] = *reinterpret_cast<const uint4*>(dst + (lane & 31) * C::PP + kq * 16 + (lane >> 5) * 8);
#pragma unroll
    for (int jj = 0; jj < C::JQ; ++jj) {
      const int j = wave + BWV * jj;
      if (j < C::NBQ)
#pragma unroll
        for (int kq = 0; kq < BT / 16; ++kq) bv[jj][kq] = tr_frag(kt, C::QP, 32 * j, kq * 16, lane);
    }
#pragma unroll
    for (int jj = 0; jj < C::JQ; ++jj) {
      const int j = wave + BWV * jj;
      if (j < C::NBQ)
#pragma unroll
        for (int kq = 0; kq < BT / 16; ++kq) dq[jj] = Mfma<IO>::m32(av[kq], bv[jj][kq], dq[jj]);
    }
  };
  // One tile in two barrier-separated phases: [S^T / dP^T of tile t, and dQ of tile t - 1]
  // then [P and dS of tile t]. K tiles, dS tiles and the token indices are double-buffered
  // (slot t & 1), so the dQ of a tile runs beside the next tile's products. Hazards: slot
  // t & 1 is rewritten at the start of tile t + 2, after every wave has passed the second
  // barrier of tile t + 1, which follows the last reads of tile t (its dQ); part is
  // rewritten by tile t + 1's products after its first barrier, which follows tile t's
  // P / dS reads of it.
  auto tile = [&](int t0, uint4 (&kreg)[KCH], int& ptok) __attribute__((always_inline)) {
    const int nv = ntok - t0 < BT ? ntok - t0 : BT;
    const int tcur = t0 / BT, sl = tcur & 1;
    uint16_t* const kt = Ks[sl];
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int idx = tid + BWV * 64 * i;
      if (idx < NCH) *reinterpret_cast<uint4*>(&kt[(idx / (C::DT / 8)) * C::QP + (idx % (C::DT / 8)) * 8]) = kreg[i];
    }
    if (tid < BT) {
      s_tok[sl][tid] = ptok;
      s_idr[(t0 / BT + 3) & 3][tid] = idreg;   // ids of tile t+3, loaded during tile t-1
      if (zf && ptok >= 0) atomicOr(&s_sel[ptok >> 5], 1u << (ptok & 31));
    }
    lds_barrier();
    load_ids(t0 + 4 * BT);
    if (t0 + 2 * BT < ntok) gather(t0 + 2 * BT, kreg, ptok);

    // ---- S^T (waves 0-3: quarters of the [nope | rope] k-range) and dP^T (waves
    // 4-7: quarters of the nope range), tokens as M, heads as N. The chain has a
    // compile-time length per role, so it is unrolled with its operand reads four
    // k-steps ahead.
    {
      auto chain = [&](auto nks_c, const uint16_t* arow) __attribute__((always_inline)) {
        constexpr int NKS = decltype(nks_c)::value;
        constexpr int AH = NKS < 4 ? NKS : 4;
        uint4 ar[AH];
#pragma unroll
        for (int i = 0; i < AH; ++i) ar[i] = *reinterpret_cast<const uint4*>(arow + i * 16);
        f32x16 sacc = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
          // pinned order (the scheduler would otherwise regroup the reads next to
          // their MFMAs): the MFMA of step ks, then the read of step ks + AH
          __builtin_amdgcn_sched_barrier(0);
          sacc = Mfma<IO>::m32(ar[ks % AH], bq[ks], sacc);
          __builtin_amdgcn_sched_barrier(0);
          if (ks + AH < NKS) ar[ks % AH] = *reinterpret_cast<const uint4*>(arow + (ks + AH) * 16);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 16; ++i) part[wave][i][lane] = sacc[i];
      };
      const uint16_t* krow = kt + (lane & 31) * C::QP + (lane >> 5) * 8;
      if (wave < 4) {
        constexpr int N = C::KS_S / 4;
        chain(std::integral_constant<int, N>{}, krow + (wave & 3) * N * 16);
      } else {
        constexpr int N = C::KS_P / 4;
        chain(std::integral_constant<int, N>{}, krow + (wave & 3) * N * 16);
      }
    }
    if (tcur > 0) dq_phase(tcur - 1);
    lds_barrier();

    // ---- P and dS of the tile (fp32 -> io dtype): dS to LDS as [head][token] for
    // dQ, both to the dense buffers (a store group = 32 heads of one token)
    constexpr int RPW = 16 / BWV;   // accumulator registers of the tile per wave
    float svs[RPW], dps[RPW];   // all partial sums requested first
#pragma unroll
    for (int j = 0; j < RPW; ++j) {
      const int i = wave * RPW + j;
      svs[j] = (part[0][i][lane] + part[1][i][lane]) + (part[2][i][lane] + part[3][i][lane]);
      dps[j] = (part[4][i][lane] + part[5][i][lane]) + (part[6][i][lane] + part[7][i][lane]);
    }
#pragma unroll
    for (int j = 0; j < RPW; ++j) {
      const int i = wave * RPW + j;
      const int tk = m32_row(i, lane), h = lane & 31;
      const float sv = svs[j];
      const float dp = dps[j];
      float p = 0.f, ds = 0.f;
      if (tk < nv && h < hn) {
        p = __builtin_amdgcn_exp2f(sv * sl2 - s_m[h]) * s_il[h];
        ds = p * (dp - s_dl[h]) * f.scale;
      }
      const uint16_t ds16 = from_f32<IO>(ds);
      dSs[sl][h * C::PP + tk] = ds16;
      const int tb = s_tok[sl][tk];
      if (tb >= 0 && h < hn) {
        const int64_t di = dbase + (int64_t)tb * g.kp + h;
        w.dst[di] = ds16;
        w.pt[di] = from_f32<IO>(p);
      }
    }
  };
  if (zf)
    for (int i = tid; i < (g.nk + 31) / 32; i += BWV * 64) s_sel[i] = 0;
  // prologue: the ids of tiles 0-2 straight to the ring, tile 3's into idreg
  if (tid < 3 * BT) s_idr[tid / BT][tid % BT] = tid < ntok ? toks[tid] : -1;
  load_ids(3 * BT);
  lds_barrier();
  if (ntok > 0) gather(0, ka, pa);
  if (ntok > BT) gather(BT, kbr, pb);
  for (int t0 = 0; t0 < ntok; t0 += 2 * BT) {
    tile(t0, ka, pa);
    if (t0 + BT < ntok) tile(t0 + BT, kbr, pb);
  }
  if (ntok > 0) {   // the last tile's dQ, after its dS is complete
    lds_barrier();
    dq_phase((ntok - 1) / BT);
  }

  // ---- d_query | d_query_rope of the block's heads (zeros for rows without tokens)
  uint16_t* dqo = reinterpret_cast<uint16_t*>(a.dq);
  uint16_t* dqro = reinterpret_cast<uint16_t*>(a.dqr);
#pragma unroll
  for (int jj = 0; jj < C::JQ; ++jj) {
    const int j = wave + BWV * jj;
    if (j < C::NBQ) {
      const int col = 32 * j + (lane & 31);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int h = m32_row(i, lane);
        if (h < hn) {
          const int64_t hr = (int64_t)r * n1 + h0 + h;
          const uint16_t v = from_f32<IO>(dq[jj][i]);
          if (col < D) dqo[hr * D + col] = v;
          else dqro[hr * BDR + (col - D)] = v;
        }
      }
    }
  }

  // ---- zeros of this (row, head block)'s dense slice at the tokens it did not write
  // (the last tile's barrier published every bit): 8 threads per token, 16 bytes of
  // one buffer each; the slice is 16-byte aligned as N1 % 8 == 0 and kp % 64 == 0
  if (zf) {
    const int q = tid & 7;
    if ((q & 3) * 8 < hn) {
      uint16_t* zb = (q < 4 ? w.dst : w.pt) + dbase + (q & 3) * 8;
      for (int t = tid >> 3; t < g.nk; t += BWV * 8)
        if (!((s_sel[t >> 5] >> (t & 31)) & 1u)) stg16(zb + (int64_t)t * g.kp, z4);
    }
  }
}

// ---- staged library-GEMM rows to the outputs: key row kr of batch b (the last batch
// with key_start[b] <= kr), t = kr - key_start[b], takes staged row boffk[b] + t when
// t < nk and the batch has query rows; every other key row is zero. One thread per 8
// elements of the [D | Dr | D] row.
template <int IO, int D>
__global__ __launch_bounds__(256) void sfa_bwd_place_kernel(SfaBwdArgs a, BwdWs w) {
  const SfaArgs& f = a.f;
  constexpr int UK = D / 8, UR = BDR / 8, U = 2 * UK + UR;   // 8-element units per key row
  const int64_t n = f.key_rows * U;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t kr = i / U;
    const int u = (int)(i - kr * U);
    int lo = 0, hi = f.batch - 1;   // last b with key_start[b] <= kr (key_start ascends)
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (f.key_start[mid] <= kr) lo = mid; else hi = mid - 1;
    }
    const int b = lo;
    const int64_t t = kr - f.key_start[b];
    const bool covered = t >= 0 && t < batch_nk(f.act_k[b], f.s2) && f.row_start[b + 1] > f.row_start[b];
    const int64_t sr = covered ? w.boffk[b] + t : 0;
    const int64_t srows = w.boffk[f.batch];   // staged rows per partial
    // the sum of the split's fp32 partials of 8 consecutive elements, in the io dtype
    auto sum8 = [&](const float* p, int64_t pstride) {
      // every partial's loads are issued before the first add (unrolled to BSPLIT)
      float4 x[BSPLIT], y[BSPLIT];
#pragma unroll
      for (int c = 0; c < BSPLIT; ++c)
        if (c < w.split) {
          x[c] = reinterpret_cast<const float4*>(p + c * pstride)[0];
          y[c] = reinterpret_cast<const float4*>(p + c * pstride)[1];
        }
      float4 lo = make_float4(0.f, 0.f, 0.f, 0.f), hi = lo;
#pragma unroll
      for (int c = 0; c < BSPLIT; ++c)
        if (c < w.split) {
          lo.x += x[c].x; lo.y += x[c].y; lo.z += x[c].z; lo.w += x[c].w;
          hi.x += y[c].x; hi.y += y[c].y; hi.z += y[c].z; hi.w += y[c].w;
        }
      return make_uint4(pack2<IO>(lo.x, lo.y), pack2<IO>(lo.z, lo.w), pack2<IO>(hi.x, hi.y), pack2<IO>(hi.z, hi.w));
    };
    uint4 v = make_uint4(0, 0, 0, 0);
    if (u < UK) {
      if (covered) v = sum8(w.skc + sr * (D + BDR) + u * 8, srows * (D + BDR));
      stg16(reinterpret_cast<uint16_t*>(a.dk) + kr * D + u * 8, v);
    } else if (u < UK + UR) {
      if (covered) v = sum8(w.skc + sr * (D + BDR) + D + (u - UK) * 8, srows * (D + BDR));
      stg16(reinterpret_cast<uint16_t*>(a.dkr) + kr * BDR + (u - UK) * 8, v);
    } else {
      if (covered) v = sum8(w.sv + sr * D + (u - UK - UR) * 8, srows * D);
      stg16(reinterpret_cast<uint16_t*>(a.dv) + kr * D + (u - UK - UR) * 8, v);
    }
  }
}

template <int IO, int D>
hipError_t launch_rows_d(const SfaBwdArgs& a, const SfaTokenLists& tl, const BwdWs& w, hipStream_t s) {
  const SfaArgs& f = a.f;
  if (f.total_rows > 0) {
    const dim3 grid(f.total_rows, (f.n1 + BH - 1) / BH);
    hipLaunchKernelGGL((sfa_bwd_rows_kernel<IO, D>), grid, dim3(BWV * 64), 0, s, a, tl, w);
  }
  return hipGetLastError();
}

template <int IO>
hipError_t launch_rows_io(const SfaBwdArgs& a, const SfaTokenLists& tl, const BwdWs& w, hipStream_t s) {
  switch (a.f.d) {
    case 128: return launch_rows_d<IO, 128>(a, tl, w, s);
    case 256: return launch_rows_d<IO, 256>(a, tl, w, s);
    case 512: return launch_rows_d<IO, 512>(a, tl, w, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_place(const SfaBwdArgs& a, const BwdWs& w, hipStream_t s) {
  const int64_t units = a.f.key_rows * (2 * a.f.d + BDR) / 8;
  if (units == 0) return hipSuccess;
  const int blocks = (int)((units + 255) / 256 < 8192 ? (units + 255) / 256 : 8192);
  const bool bf = a.f.io == IO_BF16;
  switch (a.f.d) {
    case 128:
      if (bf) hipLaunchKernelGGL((sfa_bwd_place_kernel<IO_BF16, 128>), dim3(blocks), dim3(256), 0, s, a, w);
      else hipLaunchKernelGGL((sfa_bwd_place_kernel<IO_F16, 128>), dim3(blocks), dim3(256), 0, s, a, w);
      break;
    case 256:
      if (bf) hipLaunchKernelGGL((sfa_bwd_place_kernel<IO_BF16, 256>), dim3(blocks), dim3(256), 0, s, a, w);
      else hipLaunchKernelGGL((sfa_bwd_place_kernel<IO_F16, 256>), dim3(blocks), dim3(256), 0, s, a, w);
      break;
    case 512:
      if (bf) hipLaunchKernelGGL((sfa_bwd_place_kernel<IO_BF16, 512>), dim3(blocks), dim3(256), 0, s, a, w);
      else hipLaunchKernelGGL((sfa_bwd_place_kernel<IO_F16, 512>), dim3(blocks), dim3(256), 0, s, a, w);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// ---- library GEMMs. hipBLASLt is loaded (dlopen) by the first backward call, so the
// indexer / forward library has no load-time dependency on it. One handle per device,
// created on that device's first backward call outside stream capture (the library
// allocates its own small state then). The algorithm of a product is fixed per shape: the
// entry of hipBLASLt's ranked heuristic list that a committed table names for the shape
// (measured on this image's hipBLASLt), else the list's first entry. The list is a
// deterministic function of the library build and the product's shape, so every process
// uses the same kernel and gets the same bits; nothing is timed and the host never waits.
struct LtApi {
  decltype(&hipblasLtCreate) create = nullptr;
  decltype(&hipblasLtMatmulDescCreate) desc_create = nullptr;
  decltype(&hipblasLtMatmulDescSetAttribute) desc_set = nullptr;
  decltype(&hipblasLtMatmulDescDestroy) desc_destroy = nullptr;
  decltype(&hipblasLtMatrixLayoutCreate) layout_create = nullptr;
  decltype(&hipblasLtMatrixLayoutSetAttribute) layout_set = nullptr;
  decltype(&hipblasLtMatrixLayoutDestroy) layout_destroy = nullptr;
  decltype(&hipblasLtMatmulPreferenceCreate) pref_create = nullptr;
  decltype(&hipblasLtMatmulPreferenceSetAttribute) pref_set = nullptr;
  decltype(&hipblasLtMatmulPreferenceDestroy) pref_destroy = nullptr;
  decltype(&hipblasLtMatmulAlgoGetHeuristic) heuristic = nullptr;
  decltype(&hipblasLtMatmul) matmul = nullptr;
  bool ok = false;
  std::string error;
};
const LtApi& lt_api() {
  static LtApi api;
  static std::once_flag once;
  std::call_once(once, [] {
    void* h = nullptr;
    for (const char* name : {"libhipblaslt.so.1", "libhipblaslt.so", "/opt/rocm/lib/libhipblaslt.so.1"})
      if ((h = dlopen(name, RTLD_NOW | RTLD_LOCAL)) != nullptr) break;
    if (!h) {
      const char* e = dlerror();
      api.error = std::string("hipBLASLt could not be loaded: ") + (e ? e : "libhipblaslt.so.1 not found");
      return;
    }
    bool all = true;
    auto sym = [&](auto& fn, const char* name) {
      fn = reinterpret_cast<std::remove_reference_t<decltype(fn)>>(dlsym(h, name));
      all = all && fn != nullptr;
    };
    sym(api.create, "hipblasLtCreate");
    sym(api.desc_create, "hipblasLtMatmulDescCreate");
    sym(api.desc_set, "hipblasLtMatmulDescSetAttribute");
    sym(api.desc_destroy, "hipblasLtMatmulDescDestroy");
    sym(api.layout_create, "hipblasLtMatrixLayoutCreate");
    sym(api.layout_set, "hipblasLtMatrixLayoutSetAttribute");
    sym(api.layout_destroy, "hipblasLtMatrixLayoutDestroy");
    sym(api.pref_create, "hipblasLtMatmulPreferenceCreate");
    sym(api.pref_set, "hipblasLtMatmulPreferenceSetAttribute");
    sym(api.pref_destroy, "hipblasLtMatmulPreferenceDestroy");
    sym(api.heuristic, "hipblasLtMatmulAlgoGetHeuristic");
    sym(api.matmul, "hipblasLtMatmul");
    if (!all) {
      api.error = "hipBLASLt is missing an entry point this library uses";
      return;
    }
    api.ok = true;
  });
  return api;
}

// Committed algorithm choices: the position in the heuristic's ranked list for a product
// shape (element size, output columns, key rows, contraction, dense row stride, split).
// Measured at the reference's grad perf shape (perf_sfa_grad_triton.py:23) on this image's
// hipBLASLt: the [d_key | d_key_rope] product runs 0.167 ms with entry 38 against 0.198 ms
// with the first entry; for the d_value product the first entry is within 1% of the best.
struct LtPick {
  int esize, n_cols, nk, k;
  int64_t kp;
  int split, index;
};
constexpr LtPick LT_PICKS[] = {
    {2, 576, 4096, 32768, 32768, 4, 38},
};

struct LtCache {
  std::mutex mu;
  std::map<int, hipblasLtHandle_t> handle;
  std::map<std::tuple<int, int, int, int, int, int64_t, int>, hipblasLtMatmulAlgo_t> algo;
};
LtCache& lt_cache() {
  static LtCache c;
  return c;
}

// The device's hipBLASLt handle; the first call on a device creates it and must not be
// under stream capture (hipErrorStreamCaptureUnsupported).
hipError_t lt_handle(hipStream_t s, hipblasLtHandle_t* h) {
  const LtApi& api = lt_api();
  if (!api.ok) return hipErrorSharedObjectInitFailed;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return hipErrorInvalidDevice;
  LtCache& c = lt_cache();
  std::lock_guard<std::mutex> g(c.mu);
  auto it = c.handle.find(dev);
  if (it != c.handle.end()) {
    *h = it->second;
    return hipSuccess;
  }
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cap) != hipSuccess) return hipErrorInvalidValue;
  if (cap != hipStreamCaptureStatusNone) return hipErrorStreamCaptureUnsupported;
  if (api.create(h) != HIPBLAS_STATUS_SUCCESS) return hipErrorNotInitialized;
  c.handle[dev] = *h;
  return hipSuccess;
}

// staged[c][t, col] = sum over j in chunk c of dense[t, j] b_rows[j, col] (fp32), for the
// `split` equal chunks of the contraction k, as one strided-batched product. In
// column-major terms the product of a batch is C^T [N x nk] = B^T [N x K] * A^T [K x nk]:
// B^T is the row-major [K x N] operand (q | q_rope or d_out rows of the batch, ld N), A^T
// the row-major dense [nk x kp] buffer (ld kp, its first K = nq * N1 columns), C^T the
// row-major staged [nk x N] rows (ld N).
hipError_t lt_gemm(hipDataType dt, int n_cols, int nk, int k, int split, const void* b_rows, const void* dense,
                   int64_t kp, float* staged, int64_t split_stride, void* ws, hipStream_t s) {
  const LtApi& api = lt_api();
  hipblasLtHandle_t h;
  hipError_t he = lt_handle(s, &h);
  if (he != hipSuccess) return he;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return hipErrorInvalidDevice;
  LtCache& c = lt_cache();
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
  hipblasLtMatmulPreference_t pref = nullptr;
  hipError_t ret = hipErrorNotSupported;
  const hipblasOperation_t op = HIPBLAS_OP_N;
  const uint64_t wsb = LT_WS;
  const float alpha = 1.f, beta = 0.f;
  do {
    if (api.desc_create(&desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS) break;
    if (api.desc_set(desc, HIPBLASLT_MATMUL_DESC_TRANSA, &op, sizeof(op)) != HIPBLAS_STATUS_SUCCESS ||
        api.desc_set(desc, HIPBLASLT_MATMUL_DESC_TRANSB, &op, sizeof(op)) != HIPBLAS_STATUS_SUCCESS)
      break;
    const int kc = k / split;
    if (api.layout_create(&la, dt, n_cols, kc, n_cols) != HIPBLAS_STATUS_SUCCESS ||
        api.layout_create(&lb, dt, kc, nk, kp) != HIPBLAS_STATUS_SUCCESS ||
        api.layout_create(&lc, HIP_R_32F, n_cols, nk, n_cols) != HIPBLAS_STATUS_SUCCESS)
      break;
    if (split > 1) {
      const int32_t bc = split;
      const int64_t sa = (int64_t)kc * n_cols, sb = kc, sc = split_stride;
      if (api.layout_set(la, HIPBLASLT_MATRIX_LAYOUT_BATCH_COUNT, &bc, sizeof(bc)) != HIPBLAS_STATUS_SUCCESS ||
          api.layout_set(la, HIPBLASLT_MATRIX_LAYOUT_STRIDED_BATCH_OFFSET, &sa, sizeof(sa)) != HIPBLAS_STATUS_SUCCESS ||
          api.layout_set(lb, HIPBLASLT_MATRIX_LAYOUT_BATCH_COUNT, &bc, sizeof(bc)) != HIPBLAS_STATUS_SUCCESS ||
          api.layout_set(lb, HIPBLASLT_MATRIX_LAYOUT_STRIDED_BATCH_OFFSET, &sb, sizeof(sb)) != HIPBLAS_STATUS_SUCCESS ||
          api.layout_set(lc, HIPBLASLT_MATRIX_LAYOUT_BATCH_COUNT, &bc, sizeof(bc)) != HIPBLAS_STATUS_SUCCESS ||
          api.layout_set(lc, HIPBLASLT_MATRIX_LAYOUT_STRIDED_BATCH_OFFSET, &sc, sizeof(sc)) != HIPBLAS_STATUS_SUCCESS)
        break;
    }
    hipblasLtMatmulAlgo_t algo;
    const auto key = std::make_tuple(dev, (int)dt, n_cols, nk, k, kp, split);
    bool have = false;
    {
      std::lock_guard<std::mutex> g(c.mu);
      auto it = c.algo.find(key);
      if (it != c.algo.end()) {
        algo = it->second;
        have = true;
      }
    }
    if (!have) {   // host-side query only: no GPU work, no synchronisation
      if (api.pref_create(&pref) != HIPBLAS_STATUS_SUCCESS ||
          api.pref_set(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsb, sizeof(wsb)) != HIPBLAS_STATUS_SUCCESS)
        break;
      hipblasLtMatmulHeuristicResult_t res[LT_CANDIDATES];
      int nres = 0;
      if (api.heuristic(h, desc, la, lb, lc, lc, pref, LT_CANDIDATES, res, &nres) != HIPBLAS_STATUS_SUCCESS ||
          nres < 1)
        break;
      int pick = 0;
      const int esize = 2;   // bf16 / fp16 operands
      for (const LtPick& p : LT_PICKS)
        if (p.esize == esize && p.n_cols == n_cols && p.nk == nk && p.k == k && p.kp == kp && p.split == split &&
            p.index < nres && res[p.index].workspaceSize <= LT_WS)
          pick = p.index;
      algo = res[pick].algo;
      std::lock_guard<std::mutex> g(c.mu);
      c.algo[key] = algo;
    }
    if (api.matmul(h, desc, &alpha, b_rows, la, dense, lb, &beta, staged, lc, staged, lc, &algo, ws, LT_WS, s) !=
        HIPBLAS_STATUS_SUCCESS)
      break;
    ret = hipSuccess;
  } while (false);
  if (pref) api.pref_destroy(pref);
  if (lc) api.layout_destroy(lc);
  if (lb) api.layout_destroy(lb);
  if (la) api.layout_destroy(la);
  if (desc) api.desc_destroy(desc);
  return ret;
}

// Host geometry (the device's batch_geo from the host copies): staged rows, dense
// elements and, per batch, (nq, nk, kp, dense offset, staged offset).
struct HostGeo {
  int64_t staged = 0, dense = 0;
};
HostGeo bwd_host_geo(int batch, const int32_t* h_row_start, const int32_t* h_act_k, int s2, int n1) {
  HostGeo g;
  for (int b = 0; b < batch; ++b) {
    const int nq = h_row_start[b + 1] - h_row_start[b];
    const int nk = batch_nk(h_act_k[b], s2);
    g.staged += nk;
    g.dense += (int64_t)nk * dense_row(nq, n1);
  }
  return g;
}

// Workspace: token lists | batch offsets | staged offsets | staged d_key, d_key_rope,
// d_value rows | library-GEMM workspace | dS_T | P_T. Returns the offset of dS_T; the
// two dense buffers share the rest equally.
size_t bwd_fixed_bytes(int total_rows, int batch, int topk, int sbs, int64_t staged, int d, int n1) {
  size_t off = align256(sfa_token_ws_bytes(total_rows > 0 ? total_rows : 1, topk, sbs));
  off += 2 * align256((size_t)(batch + 1) * 8);
  off += align256((size_t)BSPLIT * staged * (d + BDR) * 4);
  off += align256((size_t)BSPLIT * staged * d * 4);
  off += align256((size_t)(total_rows > 0 ? total_rows : 0) * n1 * (d + BDR) * 2);
  off += align256((size_t)(total_rows > 0 ? total_rows : 0) * n1 * d * 2);
  off += LT_WS;
  return off;
}

}  // namespace
}  // namespace dsa

size_t sfa_bwd_workspace_bytes(int batch, const int32_t* h_row_start, const int32_t* h_act_k, int s2,
                               int total_rows, int n1, int d, int topk, int sbs, int64_t key_rows) {
  (void)key_rows;
  const dsa::HostGeo g = dsa::bwd_host_geo(batch, h_row_start, h_act_k, s2, n1);
  return dsa::bwd_fixed_bytes(total_rows, batch, topk, sbs, g.staged, d, n1) + 2 * dsa::align256((size_t)g.dense * 2);
}

hipError_t launch_sfa_bwd(const SfaBwdArgs& a, hipStream_t s) {
  const SfaArgs& f = a.f;
  char* base = reinterpret_cast<char*>(f.ws);
  SfaTokenLists tl{};
  hipError_t e = launch_sfa_token_lists(f, base, &tl, s);
  if (e != hipSuccess) return e;
  const dsa::HostGeo hg = dsa::bwd_host_geo(f.batch, a.h_row_start, a.h_act_k, f.s2, f.n1);
  size_t off = dsa::align256(sfa_token_ws_bytes(f.total_rows > 0 ? f.total_rows : 1, f.topk, f.sbs));
  dsa::BwdWs w;
  w.boff = reinterpret_cast<int64_t*>(base + off);
  off += dsa::align256((size_t)(f.batch + 1) * 8);
  w.boffk = reinterpret_cast<int64_t*>(base + off);
  off += dsa::align256((size_t)(f.batch + 1) * 8);
  w.skc = reinterpret_cast<float*>(base + off);
  off += dsa::align256((size_t)dsa::BSPLIT * hg.staged * (f.d + dsa::BDR) * 4);
  w.sv = reinterpret_cast<float*>(base + off);
  off += dsa::align256((size_t)dsa::BSPLIT * hg.staged * f.d * 4);
  // the contraction split applies to every batch: each batch's (row, head) count is
  // then a multiple of BSPLIT * 64 and large enough for the split to pay
  w.split = dsa::BSPLIT;
  for (int b = 0; b < f.batch; ++b) {
    const int kb_ = (a.h_row_start[b + 1] - a.h_row_start[b]) * f.n1;
    if (dsa::batch_nk(a.h_act_k[b], f.s2) > 0 && kb_ > 0 && (kb_ % (dsa::BSPLIT * 64) != 0 || kb_ < 4096)) w.split = 1;
  }
  w.qcat = reinterpret_cast<uint16_t*>(base + off);
  off += dsa::align256((size_t)(f.total_rows > 0 ? f.total_rows : 0) * f.n1 * (f.d + dsa::BDR) * 2);
  w.gocat = reinterpret_cast<uint16_t*>(base + off);
  off += dsa::align256((size_t)(f.total_rows > 0 ? f.total_rows : 0) * f.n1 * f.d * 2);
  w.lt_ws = base + off;
  off += dsa::LT_WS;
  // the two dense buffers split what is left (256-byte aligned halves)
  const size_t rest = f.ws_bytes > off ? f.ws_bytes - off : 0;
  const size_t half = rest / 2 / 256 * 256;
  w.dst = reinterpret_cast<uint16_t*>(base + off);
  w.pt = reinterpret_cast<uint16_t*>(base + off + half);
  w.cap = (int64_t)(half / 2);
  if (hg.dense > w.cap) return hipErrorInvalidValue;   // the caller's workspace is checked against this size
  // the rows kernel writes the zeros itself when every batch's tokens fit its bitmap
  // and the (row, head block) slices are 16-byte aligned
  int max_nk = 0;
  for (int b = 0; b < f.batch; ++b) {
    const int nk = dsa::batch_nk(a.h_act_k[b], f.s2);
    max_nk = nk > max_nk ? nk : max_nk;
  }
  const int zbw = f.d == 128 ? dsa::BCfg<128>::ZBW : (f.d == 256 ? dsa::BCfg<256>::ZBW : dsa::BCfg<512>::ZBW);
  w.zfuse = f.n1 % 8 == 0 && (int64_t)max_nk <= 32 * (int64_t)zbw;

  hipLaunchKernelGGL(dsa::sfa_bwd_geo_kernel, dim3(1), dim3(256), 0, s, f, w);
  if (!w.zfuse) {
    const int zb = 2048;
    hipLaunchKernelGGL(dsa::sfa_bwd_zero_kernel, dim3(zb), dim3(256), 0, s, reinterpret_cast<uint4*>(w.dst),
                       (int64_t)(half / 16), (const int64_t*)(w.boff + f.batch), w.cap);
    hipLaunchKernelGGL(dsa::sfa_bwd_zero_kernel, dim3(zb), dim3(256), 0, s, reinterpret_cast<uint4*>(w.pt),
                       (int64_t)(half / 16), (const int64_t*)(w.boff + f.batch), w.cap);
  }
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  e = f.io == dsa::IO_BF16 ? dsa::launch_rows_io<dsa::IO_BF16>(a, tl, w, s)
                           : dsa::launch_rows_io<dsa::IO_F16>(a, tl, w, s);
  if (e != hipSuccess) return e;
  // the two products of every batch holding query rows and key tokens
  const hipDataType dt = f.io == dsa::IO_BF16 ? HIP_R_16BF : HIP_R_16F;
  int64_t doff = 0, soff = 0;
  for (int b = 0; b < f.batch; ++b) {
    const int rs = a.h_row_start[b], nq = a.h_row_start[b + 1] - rs;
    const int nk = dsa::batch_nk(a.h_act_k[b], f.s2);
    const int kp = dsa::dense_row(nq, f.n1);
    const int k = nq * f.n1;
    if (nk > 0 && k > 0) {
      const int64_t brow = (int64_t)rs * f.n1;
      const int dt_w = f.d + dsa::BDR;
      if ((e = dsa::lt_gemm(dt, dt_w, nk, k, w.split, w.qcat + brow * dt_w, w.dst + doff, kp, w.skc + soff * dt_w,
                            hg.staged * dt_w, w.lt_ws, s)) != hipSuccess ||
          (e = dsa::lt_gemm(dt, f.d, nk, k, w.split, w.gocat + brow * f.d, w.pt + doff, kp, w.sv + soff * f.d,
                            hg.staged * f.d, w.lt_ws, s)) != hipSuccess)
        return e;
    }
    doff += (int64_t)nk * kp;
    soff += nk;
  }
  return dsa::launch_place(a, w, s);
}

const char* sfa_bwd_library_error() { return dsa::lt_api().error.c_str(); }
