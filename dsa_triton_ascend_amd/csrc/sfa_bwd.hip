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
//  3. sfa_bwd_rows_kernel -- one work-group (4 waves) per (query row, block of
//     32 heads). Q | Q rope and dO of the block sit in LDS for the whole row; the
//     row's tokens are processed in tiles of 32 gathered [D | Dr] rows:
//       * S^T = K Q^T and dP^T = K_nope dO^T on v_mfma_f32_32x32x16 (tokens as
//         M, heads as N), their k-ranges split over the four waves and summed
//         through LDS;
//       * P and dS in fp32, stored in the io dtype to the dense buffers (32
//         consecutive heads of one token per store group) and dS also to LDS as
//         [head][token];
//       * dQ[head, col] += dS K, each wave owning a quarter of the 32-column
//         blocks, the K operand read with ds_read_b64_tr_b16 from the tile;
//  4. sfa_bwd_gemm_kernel (twice: d_key | d_key_rope, d_value) -- 128 x BN
//     output tiles per batch on v_mfma_f32_32x32x16, operands streamed with
//     direct-to-LDS loads through a 3-stage LDS ring two k-steps ahead, the k-range
//     split over work-groups when the tiles alone do not fill the GPU; partial tiles are
//     added into fp32 accumulators with global atomics (so the last bits may
//     differ from run to run, the reference's deterministic=False contract,
//     sparse_flash_attention_grad_triton.py:550);
//  5. sfa_bwd_finish_kernel -- converts the accumulators to the io dtype.
#include <climits>

#include "dsa_common.hpp"

namespace dsa {
namespace {

constexpr int BDR = 64;     // rope width
constexpr int BH = 32;      // heads per work-group (rows kernel)
constexpr int BT = 32;      // tokens per tile
constexpr int BWV = 4;      // waves per work-group
constexpr float BLOG2E = 1.4426950408889634f;
constexpr int GBM = 128;    // GEMM tile rows (key tokens)
constexpr int GBK = 64;     // GEMM k-step; dense rows are padded to a multiple of it

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
  static_assert(KS_S % 2 == 0 && KS_P % 2 == 0, "k-ranges split in halves");
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
  float* dk;       // [key_rows, D]   fp32 accumulators
  float* dkr;      // [key_rows, Dr]
  float* dv;       // [key_rows, D]
  uint16_t* dst;   // dS_T dense buffer (io dtype)
  uint16_t* pt;    // P_T dense buffer (io dtype)
  int64_t cap;     // elements per dense buffer
};

// Dense geometry of batch b: query rows [rs, rs + nq), key rows [ks, ks + nk)
// (the tokens a row of the batch can select, t < min(act_k, S2)), dense rows of
// kp = nq * N1 rounded up to GBK elements.
struct BatchGeo {
  int rs, nq, ks, nk, kp;
};

__host__ __device__ inline int dense_row(int nq, int n1) { return (nq * n1 + GBK - 1) / GBK * GBK; }

__device__ __forceinline__ BatchGeo batch_geo(const SfaArgs& f, int b) {
  BatchGeo g;
  g.rs = f.row_start[b];
  g.nq = f.row_start[b + 1] - g.rs;
  g.ks = f.key_start[b];
  int nk = f.act_k[b] < f.s2 ? f.act_k[b] : f.s2;
  const int64_t room = f.key_rows - g.ks;
  nk = nk < 0 ? 0 : nk;
  g.nk = (int64_t)nk < room ? nk : (int)(room > 0 ? room : 0);
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
  __shared__ __attribute__((aligned(16))) uint16_t Qs[BH * C::QP];    // [head][nope | rope]
  __shared__ __attribute__((aligned(16))) uint16_t Ks[BT * C::QP];    // [token][nope | rope]
  __shared__ __attribute__((aligned(16))) uint16_t dOs[BH * C::OP];   // [head][D]
  __shared__ __attribute__((aligned(16))) uint16_t dSs[BH * C::PP];   // [head][token]
  __shared__ float part[BWV][16][64];   // S^T / dP^T k-range partials, MFMA layout
  __shared__ int s_tok[BT];             // the tile's token index within the batch (-1: none)
  __shared__ int s_idr[4][BT];          // token-id ring: the ids of tile t in slot t % 4
  __shared__ float s_m[BH], s_il[BH], s_dl[BH];

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

  // ---- the block's Q | Q rope and dO (rows past the heads are zero), stats
  {
    const uint16_t* qb = reinterpret_cast<const uint16_t*>(f.q);
    const uint16_t* qrb = reinterpret_cast<const uint16_t*>(f.qr);
    const uint16_t* gob = reinterpret_cast<const uint16_t*>(a.d_out);
    for (int i = tid; i < BH * (C::DT / 8); i += BWV * 64) {
      const int h = i / (C::DT / 8), c = (i % (C::DT / 8)) * 8;
      uint4 v = z4;
      if (h < hn) {
        const int64_t hr = (int64_t)r * n1 + h0 + h;
        v = c < D ? ldg16(qb + hr * D + c) : ldg16(qrb + hr * BDR + (c - D));
      }
      *reinterpret_cast<uint4*>(&Qs[h * C::QP + c]) = v;
    }
    for (int i = tid; i < BH * (D / 8); i += BWV * 64) {
      const int h = i / (D / 8), c = (i % (D / 8)) * 8;
      const uint4 v = h < hn ? ldg16(gob + ((int64_t)r * n1 + h0 + h) * D + c) : z4;
      *reinterpret_cast<uint4*>(&dOs[h * C::OP + c]) = v;
    }
    // delta = dO . O (fp32) per head: 8 threads per head, D/8 columns each
    const uint16_t* ob = reinterpret_cast<const uint16_t*>(a.out);
    const int h = tid >> 3, part8 = tid & 7;
    float dl = 0.f;
    if (h < hn) {
      const int64_t hr = (int64_t)r * n1 + h0 + h;
      for (int c = part8 * 8; c < D; c += 64) {
        const uint4 o = ldg16(ob + hr * D + c), gv = ldg16(gob + hr * D + c);
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
    if (part8 == 0) {
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

  // ---- gathers of a tile's [nope | rope] rows into registers (rows outside the key
  // tensors and slots past the list are zero), two register sets: the next two
  // tiles' rows are in flight while one is computed
  constexpr int KCH = BT * (C::DT / 8) / (BWV * 64);   // 16-byte chunks per thread
  static_assert(KCH * BWV * 64 == BT * (C::DT / 8), "tile splits evenly");
  uint4 ka[KCH], kbr[KCH];
  int pa = -1, pb = -1;
  auto gather = [&](int t0, uint4 (&kreg)[KCH], int& ptok) __attribute__((always_inline)) {
    const int nvt = ntok - t0 < BT ? ntok - t0 : BT;
    const int* ids = s_idr[(t0 / BT) & 3];
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int idx = tid + BWV * 64 * i;
      const int t = idx / (C::DT / 8), c = (idx % (C::DT / 8)) * 8;
      const int p = t < nvt ? ids[t] : -1;
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
  auto tile = [&](int t0, uint4 (&kreg)[KCH], int& ptok) __attribute__((always_inline)) {
    const int nv = ntok - t0 < BT ? ntok - t0 : BT;
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int idx = tid + BWV * 64 * i;
      *reinterpret_cast<uint4*>(&Ks[(idx / (C::DT / 8)) * C::QP + (idx % (C::DT / 8)) * 8]) = kreg[i];
    }
    if (tid < BT) {
      s_tok[tid] = ptok;
      s_idr[(t0 / BT + 3) & 3][tid] = idreg;   // ids of tile t+3, loaded during tile t-1
    }
    lds_barrier();
    load_ids(t0 + 4 * BT);
    if (t0 + 2 * BT < ntok) gather(t0 + 2 * BT, kreg, ptok);

    // ---- S^T (waves 0, 1: halves of the [nope | rope] k-range) and dP^T (waves 2,
    // 3: halves of the nope range), tokens as M, heads as N
    {
      const bool is_s = wave < 2;
      const int nks = is_s ? C::KS_S / 2 : C::KS_P / 2;
      const int ks0 = (wave & 1) * nks;
      const uint16_t* arow = Ks + (lane & 31) * C::QP + (lane >> 5) * 8 + ks0 * 16;
      const uint16_t* brow = (is_s ? Qs + (lane & 31) * C::QP : dOs + (lane & 31) * C::OP) + (lane >> 5) * 8 + ks0 * 16;
      f32x16 sacc = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      for (int ks = 0; ks < nks; ++ks)
        sacc = Mfma<IO>::m32(*reinterpret_cast<const uint4*>(arow + ks * 16),
                             *reinterpret_cast<const uint4*>(brow + ks * 16), sacc);
#pragma unroll
      for (int i = 0; i < 16; ++i) part[wave][i][lane] = sacc[i];
    }
    lds_barrier();

    // ---- P and dS of the tile (fp32 -> io dtype): dS to LDS as [head][token] for
    // dQ, both to the dense buffers (a store group = 32 heads of one token)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = wave * 4 + j;
      const int tk = m32_row(i, lane), h = lane & 31;
      const float sv = part[0][i][lane] + part[1][i][lane];
      const float dp = part[2][i][lane] + part[3][i][lane];
      float p = 0.f, ds = 0.f;
      if (tk < nv && h < hn) {
        p = __builtin_amdgcn_exp2f(sv * sl2 - s_m[h]) * s_il[h];
        ds = p * (dp - s_dl[h]) * f.scale;
      }
      const uint16_t ds16 = from_f32<IO>(ds);
      dSs[h * C::PP + tk] = ds16;
      const int tb = s_tok[tk];
      if (tb >= 0 && h < hn) {
        const int64_t di = dbase + (int64_t)tb * g.kp + h;
        w.dst[di] = ds16;
        w.pt[di] = from_f32<IO>(p);
      }
    }
    lds_barrier();

    // ---- dQ[head, col] += dS[head, token] K[token, col]   (this wave's column blocks)
#pragma unroll
    for (int jj = 0; jj < C::JQ; ++jj) {
      const int j = wave + BWV * jj;
      if (j < C::NBQ) {
#pragma unroll
        for (int kq = 0; kq < BT / 16; ++kq) {
          const uint4 av = *reinterpret_cast<const uint4*>(dSs + (lane & 31) * C::PP + kq * 16 + (lane >> 5) * 8);
          dq[jj] = Mfma<IO>::m32(av, tr_frag(Ks, C::QP, 32 * j, kq * 16, lane), dq[jj]);
        }
      }
    }
    lds_barrier();   // the next tile overwrites Ks, dSs and s_tok
  };
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
}

// ---- dense GEMM per batch: C[t, n] = sum_k A[t, k] B[k, n] over the batch's
// (row, head) pairs k. A: the dense dS_T (KV = false: d_key | d_key_rope, B = q |
// q_rope) or P_T (KV = true: d_value, B = d_out) buffer; 128 x BN tiles, BN = 64 NB,
// four waves as 2 (rows) x 2 (columns), each 64 x 32 NB. xt = m-tile * n-tiles +
// n-tile, blockIdx.y = batch, blockIdx.z = k-split. Results are added to the fp32
// accumulators (rows t < nk of the batch).
template <int IO, int D, bool KV, int NB, int NST>
__device__ __forceinline__ void gemm_tile(const SfaBwdArgs& a, const BwdWs& w, int ksplit, int xt,
                                          uint8_t* lds) {
  constexpr int N = KV ? D : D + BDR;
  constexpr int BN = 64 * NB;
  constexpr int NT = N / BN;
  static_assert(N % BN == 0, "n-tiles cover the columns");
  constexpr int AP = GBK + 8;          // A tile pitch (elements): 8 data chunks + 1 pad chunk per row
  constexpr int BP = BN + 8;           // B tile pitch: 8 NB data chunks + 1 pad chunk
  constexpr int ACR = AP / 8, BCR = BP / 8;            // 16-byte chunk slots per row
  constexpr int NIA = GBM * ACR / 64, NIB = GBK * BCR / 64;   // 64-slot load instructions per k-step
  static_assert(NIA * 64 == GBM * ACR && NIB * 64 == GBK * BCR, "slots fill whole instructions");
  constexpr int NI = NIA + NIB;
  constexpr int NMIN = NI / BWV;       // loads per wave per k-step, at least
  constexpr int ABYTES = GBM * AP * 2, STAGE = ABYTES + GBK * BP * 2;
  const SfaArgs& f = a.f;
  const int b = blockIdx.y;
  const BatchGeo g = batch_geo(f, b);
  // xt -> (m-tile, n-tile): the NT tiles of an m-tile get x values 8 apart, so with
  // round-robin dispatch over the 8 XCDs they run on one XCD and share its L2 copy
  // of the A rows
  const int grp = xt / (8 * NT), rem = xt % (8 * NT);
  const int nt = rem / 8, mt = grp * 8 + rem % 8;
  const int m0 = mt * GBM;
  if (nt >= NT || m0 >= g.nk || w.boff[b + 1] > w.cap) return;
  const int kper = ((g.kp + ksplit - 1) / ksplit + GBK - 1) / GBK * GBK;
  const int kbeg = blockIdx.z * kper;
  const int kend = kbeg + kper < g.kp ? kbeg + kper : g.kp;
  if (kbeg >= kend) return;
  const int nsteps = (kend - kbeg) / GBK;
  const int kreal = g.nq * f.n1;   // k past this is padding: zero A columns, B rows clamped

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const uint16_t* abuf = (KV ? w.pt : w.dst) + w.boff[b];
  const uint16_t* bq = reinterpret_cast<const uint16_t*>(KV ? a.d_out : a.f.q);
  const uint16_t* bqr = reinterpret_cast<const uint16_t*>(a.f.qr);
  const int64_t brow0 = (int64_t)g.rs * f.n1;   // B row of k = 0

  // ---- k-step s goes global -> LDS stage s % NST with direct-to-LDS 16-byte loads:
  // instruction q of the step fills slots [64 q, 64 q + 64) of the tile (A slots
  // first, then B), slot = row * chunks-per-row + chunk; the pad chunk of a row
  // re-reads its chunk 0. Every address is in bounds: A rows past the batch's tokens
  // read its last token (their outputs are discarded), B rows past the batch's
  // (row, head) pairs read its last pair (they meet zero A columns). Instructions
  // are dealt round-robin to the waves; steps past the range re-load the last one,
  // so each wave issues the same loads every step.
  auto issue = [&](int step) __attribute__((always_inline)) {
    const int st = step < nsteps ? step : nsteps - 1;
    const int k0 = kbeg + st * GBK;
    uint8_t* stage = lds + (step % NST) * STAGE;
    for (int q = wave; q < NI; q += BWV) {
      const int slot = (q < NIA ? q : q - NIA) * 64 + lane;
      const void* src;
      if (q < NIA) {
        const int row = slot / ACR, ch = slot % ACR;
        int t = m0 + row;
        t = t < g.nk ? t : g.nk - 1;
        src = abuf + (int64_t)t * g.kp + k0 + (ch < 8 ? ch : 0) * 8;
      } else {
        const int row = slot / BCR, ch = slot % BCR;
        int k = k0 + row;
        k = k < kreal ? k : kreal - 1;
        const int n = nt * BN + (ch < 8 * NB ? ch : 0) * 8;
        const int64_t r = brow0 + k;
        src = (KV || n < D) ? (const void*)(bq + r * D + n) : (const void*)(bqr + r * BDR + (n - D));
      }
      lds_dma16_untracked(src, stage + (q < NIA ? q * 1024 : ABYTES + (q - NIA) * 1024));
    }
  };

  f32x16 acc[2][NB];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

#pragma unroll
  for (int s = 0; s < NST - 1; ++s) issue(s);
  for (int s = 0; s < nsteps; ++s) {
    // this wave's loads of step s have landed (the later NST - 2 steps may be in
    // flight), then every wave's (the barrier also ends step s - 1's reads of the
    // stage that the next issue refills)
    wait_vmcnt<(NST - 2) * NMIN>();
    lds_barrier();
    issue(s + NST - 1);
    const uint16_t* As = reinterpret_cast<const uint16_t*>(lds + (s % NST) * STAGE);
    const uint16_t* Bs = reinterpret_cast<const uint16_t*>(lds + (s % NST) * STAGE + ABYTES);
#pragma unroll
    for (int ks = 0; ks < GBK / 16; ++ks) {
      uint4 af[2], bfr[NB];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        af[i] = *reinterpret_cast<const uint4*>(&As[(64 * wm + 32 * i + (lane & 31)) * AP + ks * 16 + (lane >> 5) * 8]);
#pragma unroll
      for (int j = 0; j < NB; ++j) bfr[j] = tr_frag(Bs, BP, 32 * NB * wn + 32 * j, ks * 16, lane);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[i][j] = Mfma<IO>::m32(af[i], bfr[j], acc[i][j]);
    }
  }
  wait_vmcnt<0>();   // the trailing re-loads land before the work-group's LDS is released

  // ---- add the tile to the accumulators (rows past the batch's tokens skipped)
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int n = nt * BN + 32 * NB * wn + 32 * j + (lane & 31);
      float* dst = KV ? w.dv + n : (n < D ? w.dk + n : w.dkr + (n - D));
      const int ld = (KV || n < D) ? D : BDR;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int t = m0 + 64 * wm + 32 * i + m32_row(e, lane);
        if (t < g.nk) unsafeAtomicAdd(dst + (int64_t)(g.ks + t) * ld, acc[i][j][e]);
      }
    }
}

// n-tile widths (in 64-column units) of the two GEMMs: d_key | d_key_rope spans
// D + 64 columns (3, 5, 9 units), d_value D (2, 4, 8)
template <int D> struct GemmNB;
template <> struct GemmNB<128> { static constexpr int K = 3, V = 2; };
template <> struct GemmNB<256> { static constexpr int K = 5, V = 4; };
template <> struct GemmNB<512> { static constexpr int K = 3, V = 4; };

// LDS ring depth: three stages (loads two k-steps ahead) when they fit
template <int NB> struct GemmStages {
  static constexpr int STAGE = GBM * (GBK + 8) * 2 + GBK * (64 * NB + 8) * 2;
  static constexpr int NST = 3 * STAGE <= 160 * 1024 ? 3 : 2;
};

// One product per launch (d_key | d_key_rope, then d_value): each instance gets only
// the registers its tile needs.
template <int IO, int D, bool KV>
__global__ __launch_bounds__(256) void sfa_bwd_gemm_kernel(SfaBwdArgs a, BwdWs w, int ksplit) {
  constexpr int NB = KV ? GemmNB<D>::V : GemmNB<D>::K;
  using S = GemmStages<NB>;
  __shared__ __attribute__((aligned(16))) uint8_t lds[S::NST * S::STAGE];
  gemm_tile<IO, D, KV, NB, S::NST>(a, w, ksplit, blockIdx.x, lds);
}

// fp32 accumulator -> io dtype, 4 elements per step (every length is a multiple of 4)
template <int IO>
__global__ void sfa_bwd_finish_kernel(const float4* src, uint2* dst, int64_t n4) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (int64_t)gridDim.x * blockDim.x) {
    const float4 v = src[i];
    dst[i] = make_uint2(pack2<IO>(v.x, v.y), pack2<IO>(v.z, v.w));
  }
}

template <int IO, int D>
hipError_t launch_bwd_d(const SfaBwdArgs& a, const SfaTokenLists& tl, const BwdWs& w, hipStream_t s) {
  const SfaArgs& f = a.f;
  if (f.total_rows > 0) {
    const dim3 grid(f.total_rows, (f.n1 + BH - 1) / BH);
    hipLaunchKernelGGL((sfa_bwd_rows_kernel<IO, D>), grid, dim3(BWV * 64), 0, s, a, tl, w);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // GEMM grid: every (m-tile, n-tile) of the largest batch; the k-range is split so
    // each product fills about one round of one work-group per CU
    constexpr int NTK = (D + BDR) / (64 * GemmNB<D>::K), NTV = D / (64 * GemmNB<D>::V);
    const int mts = (f.s2 + GBM - 1) / GBM;
    if (mts > 0) {
      const int mts8 = (mts + 7) / 8 * 8;   // x covers whole groups of 8 m-tiles
      auto splits = [&](int nt) {
        const int64_t tiles = (int64_t)f.batch * mts * nt;
        const int64_t k = 256 / tiles;
        return (int)(k < 1 ? 1 : (k > 16 ? 16 : k));
      };
      const int kk = splits(NTK), kv = splits(NTV);
      hipLaunchKernelGGL((sfa_bwd_gemm_kernel<IO, D, false>), dim3(mts8 * NTK, f.batch, kk), dim3(256), 0, s,
                         a, w, kk);
      hipLaunchKernelGGL((sfa_bwd_gemm_kernel<IO, D, true>), dim3(mts8 * NTV, f.batch, kv), dim3(256), 0, s,
                         a, w, kv);
      e = hipGetLastError();
      if (e != hipSuccess) return e;
    }
  }
  const int64_t kr = f.key_rows;
  const struct { const float* src; void* dst; int64_t n; } outs[3] = {
      {w.dk, a.dk, kr * D}, {w.dkr, a.dkr, kr * BDR}, {w.dv, a.dv, kr * D}};
  for (const auto& o : outs) {
    if (o.n == 0) continue;
    const int64_t n4 = o.n / 4;
    const int blocks = (int)((n4 + 255) / 256 < 4096 ? (n4 + 255) / 256 : 4096);
    hipLaunchKernelGGL((sfa_bwd_finish_kernel<IO>), dim3(blocks), dim3(256), 0, s,
                       reinterpret_cast<const float4*>(o.src), reinterpret_cast<uint2*>(o.dst), n4);
  }
  return hipGetLastError();
}

template <int IO>
hipError_t launch_bwd_io(const SfaBwdArgs& a, const SfaTokenLists& tl, const BwdWs& w, hipStream_t s) {
  switch (a.f.d) {
    case 128: return launch_bwd_d<IO, 128>(a, tl, w, s);
    case 256: return launch_bwd_d<IO, 256>(a, tl, w, s);
    case 512: return launch_bwd_d<IO, 512>(a, tl, w, s);
  }
  return hipErrorInvalidValue;
}

// Workspace: token lists | batch offsets | fp32 accumulators (d_key, d_key_rope,
// d_value) | dS_T | P_T. Returns the offset of dS_T; the two dense buffers share
// the rest equally.
size_t bwd_fixed_bytes(int total_rows, int batch, int topk, int sbs, int64_t key_rows, int d) {
  size_t off = align256(sfa_token_ws_bytes(total_rows > 0 ? total_rows : 1, topk, sbs));
  off += align256((size_t)(batch + 1) * 8);
  off += align256((size_t)key_rows * d * 4);
  off += align256((size_t)key_rows * BDR * 4);
  off += align256((size_t)key_rows * d * 4);
  return off;
}

}  // namespace
}  // namespace dsa

size_t sfa_bwd_workspace_bytes(int batch, const int32_t* h_row_start, const int32_t* h_act_k, int s2,
                               int total_rows, int n1, int d, int topk, int sbs, int64_t key_rows) {
  int64_t dense = 0;
  for (int b = 0; b < batch; ++b) {
    const int nq = h_row_start[b + 1] - h_row_start[b];
    int nk = h_act_k[b] < s2 ? h_act_k[b] : s2;
    nk = nk < 0 ? 0 : nk;
    dense += (int64_t)nk * dsa::dense_row(nq, n1);
  }
  return dsa::bwd_fixed_bytes(total_rows, batch, topk, sbs, key_rows, d) + 2 * dsa::align256((size_t)dense * 2);
}

hipError_t launch_sfa_bwd(const SfaBwdArgs& a, hipStream_t s) {
  const SfaArgs& f = a.f;
  char* base = reinterpret_cast<char*>(f.ws);
  SfaTokenLists tl{};
  hipError_t e = launch_sfa_token_lists(f, base, &tl, s);
  if (e != hipSuccess) return e;
  size_t off = dsa::align256(sfa_token_ws_bytes(f.total_rows > 0 ? f.total_rows : 1, f.topk, f.sbs));
  dsa::BwdWs w;
  w.boff = reinterpret_cast<int64_t*>(base + off);
  off += dsa::align256((size_t)(f.batch + 1) * 8);
  char* acc0 = base + off;
  w.dk = reinterpret_cast<float*>(base + off);
  off += dsa::align256((size_t)f.key_rows * f.d * 4);
  w.dkr = reinterpret_cast<float*>(base + off);
  off += dsa::align256((size_t)f.key_rows * dsa::BDR * 4);
  w.dv = reinterpret_cast<float*>(base + off);
  off += dsa::align256((size_t)f.key_rows * f.d * 4);
  const size_t acc_bytes = (size_t)(base + off - acc0);
  // the two dense buffers split what is left (256-byte aligned halves)
  const size_t rest = f.ws_bytes > off ? f.ws_bytes - off : 0;
  const size_t half = rest / 2 / 256 * 256;
  w.dst = reinterpret_cast<uint16_t*>(base + off);
  w.pt = reinterpret_cast<uint16_t*>(base + off + half);
  w.cap = (int64_t)(half / 2);

  hipLaunchKernelGGL(dsa::sfa_bwd_geo_kernel, dim3(1), dim3(256), 0, s, f, w);
  const int zb = 2048;
  hipLaunchKernelGGL(dsa::sfa_bwd_zero_kernel, dim3(zb), dim3(256), 0, s, reinterpret_cast<uint4*>(acc0),
                     (int64_t)(acc_bytes / 16), (const int64_t*)nullptr, (int64_t)0);
  hipLaunchKernelGGL(dsa::sfa_bwd_zero_kernel, dim3(zb), dim3(256), 0, s, reinterpret_cast<uint4*>(w.dst),
                     (int64_t)(half / 16), (const int64_t*)(w.boff + f.batch), w.cap);
  hipLaunchKernelGGL(dsa::sfa_bwd_zero_kernel, dim3(zb), dim3(256), 0, s, reinterpret_cast<uint4*>(w.pt),
                     (int64_t)(half / 16), (const int64_t*)(w.boff + f.batch), w.cap);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  return f.io == dsa::IO_BF16 ? dsa::launch_bwd_io<dsa::IO_BF16>(a, tl, w, s)
                              : dsa::launch_bwd_io<dsa::IO_F16>(a, tl, w, s);
}
