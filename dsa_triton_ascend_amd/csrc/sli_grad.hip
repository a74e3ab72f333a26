// Sparse lightning-indexer grad KL loss for gfx950.
//
// Semantics: sli_grad_kl_loss_numpy.py:17-180 with the row bounds of
// sparse_lightning_indexer_grad_kl_loss_triton.py:63-69 (BSND, N2 = Nidx2 = 1).
// Per query row r = (b, s1 < act_q), the first n = min(topK, max(act_k - act_q +
// s1 + 1, 0)) slots of sparse_indices[r], each id clipped to [0, S2 - 1]:
//   teacher p[k] = (1/N1) sum_h exp(score[h,k] - sm_max[h]) / (sm_sum[h] + 1e-8)
//   student I[k] = sum_g w[g] relu(qi[g] . ki[k]),  sI = softmax(I) (+1e-8)
//   dI = sI - p;  loss = sum_rows sum_k p~ (log p~ - log sI~)  (x~ = max(x, 1e-8))
//   dW[g] = sum_k relu[g,k] dI[k];  ds[g,k] = dI[k] w[g] [relu > 0]
//   dQI[g] = sum_k ds[g,k] ki[k];   dKI[id_k] += sum_g ds[g,k] qi[g]  (per slot)
//
// Launches:
//  1. sli_zero_kernel -- clears the teacher sums and the fp32 dKI accumulator;
//  2. sli_teacher_kernel -- one work-group per (row, 32-head block): Q | Q rope of
//     the block in LDS, tiles of 32 gathered [D | Dr] key rows, S^T on
//     v_mfma_f32_32x32x16 (k-range split over the 4 waves, summed through LDS),
//     the block's probabilities summed over its heads and added to p[r, k];
//  3. sli_student_kernel -- one work-group per row: qi in LDS, two passes over
//     tiles of 32 gathered ki rows on 32x32x16 MFMAs (I, then softmax / dI / loss,
//     then dW, dQI in registers and dKI added per slot with fp32 atomics);
//  4. sli_finish_kernel -- dKI to the io dtype and the loss (sum of the row
//     losses, in row order).
#include <climits>

#include "dsa_common.hpp"

namespace dsa {
namespace {

constexpr int SBH = 32;     // heads per teacher work-group
constexpr int SBT = 32;     // tokens per tile
constexpr int SWV = 4;      // waves per work-group
constexpr float SEPS = 1e-8f;
constexpr float SLOG2E = 1.4426950408889634f;
constexpr int DR_TEACH = 64;       // rope width of the attention-path teacher
constexpr int SLI_MAX_TOPK = 2048;   // sparse slots per row
constexpr int SLI_MAX_SLOTS = 4096;  // student keeps the row's I / dI in LDS (dense: S2)
constexpr int SLI_MAX_GD = 64 * 512; // Nidx1 (padded to 32) x D_idx held in LDS

inline size_t salign(size_t x) { return (x + 255) & ~(size_t)255; }

struct SliArgs {
  const void* q; const void* k; const void* qr; const void* kr;
  const void* qi; const void* ki; const void* w; int io, wdt;
  const int32_t* sidx; int topk;
  const float* sm_max; const float* sm_sum;
  const int32_t* act_q; const int32_t* act_k;
  int batch, s1, s2, n1, d, dr, nidx1, didx; float scale;
  void* dqi; void* dki; void* dw; float* loss;
  float* p;        // [rows, topk] teacher sums
  float* dki_acc;  // [batch * s2, didx]
  float* row_loss; // [rows]
  float* ibuf;     // [rows, topk] I / dI when a row has more than SLI_MAX_SLOTS slots
  void* tok_ws;    // token lists of the attention-path teacher (sfa_token_ws_bytes(rows, topk, 1))
  // dense mode (sidx == nullptr: slot t is key t, up to S2 slots per row)
  int n2;                              // key heads of the teacher, stats [B, N2, S1, N1 / N2]
  const float* imax; const float* isum; // given indexer softmax stats [rows], or nullptr
  float* lse_max; float* lse_sum;       // set: the student only writes the stats
  int dki_km;      // dKI from sli_dki_km_kernel: the student leaves dI per key in dib
  float* dib;      // [rows, dib_ld] dI per (row, key): p itself in dense mode, else a zeroed
  int dib_ld;      // buffer the student adds each slot's dI into (repeated keys add)
};


__device__ __forceinline__ int row_slots(const SliArgs& a, int r, int& b, int& s1) {
  b = r / a.s1;
  s1 = r - b * a.s1;
  const int aq = a.act_q[b], ak = a.act_k[b];
  if (s1 >= aq) return 0;
  int n = ak - aq + s1 + 1;
  n = n < 0 ? 0 : n;
  return n < a.topk ? n : a.topk;
}

__device__ __forceinline__ int clip_id(int id, int s2) { return id < 0 ? 0 : (id > s2 - 1 ? s2 - 1 : id); }
__device__ __forceinline__ int slot_key(const SliArgs& a, const int32_t* ids, int t) {
  return ids ? clip_id(ids[t], a.s2) : t;
}

__device__ __forceinline__ float ld_w(const void* w, int wdt, int64_t i) {
  if (wdt == DSA_DTYPE_F32) return reinterpret_cast<const float*>(w)[i];
  const uint16_t h = reinterpret_cast<const uint16_t*>(w)[i];
  return wdt == DSA_DTYPE_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
}

__global__ void sli_zero_kernel(float4* p, int64_t n4) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = make_float4(0.f, 0.f, 0.f, 0.f);
}

// ---------------------------------------------------------------- teacher
template <int IO, int DT>
__global__ __launch_bounds__(SWV * 64) void sli_teacher_kernel(SliArgs a) {
  constexpr int QP = DT + 8;          // row pitch: odd count of 16-byte units
  constexpr int KS = DT / 16;         // k-steps
  static_assert(KS % SWV == 0, "k-range splits over the waves");
  __shared__ __attribute__((aligned(16))) uint16_t Qs[SBH * QP];
  __shared__ __attribute__((aligned(16))) uint16_t Ks[SBT * QP];
  __shared__ float part[SWV][16][64];
  __shared__ float s_m[SBH], s_il[SBH];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = blockIdx.x;
  int b, s1;
  const int n = row_slots(a, r, b, s1);
  if (n == 0) return;
  const int h0 = blockIdx.y * SBH;
  const int hn = a.n1 - h0 < SBH ? a.n1 - h0 : SBH;
  const int D = a.d;
  const uint16_t* qb = reinterpret_cast<const uint16_t*>(a.q);
  const uint16_t* qrb = reinterpret_cast<const uint16_t*>(a.qr);
  const uint16_t* kb = reinterpret_cast<const uint16_t*>(a.k);
  const uint16_t* krb = reinterpret_cast<const uint16_t*>(a.kr);
  const uint4 z4 = make_uint4(0, 0, 0, 0);
  for (int i = tid; i < SBH * (DT / 8); i += SWV * 64) {
    const int h = i / (DT / 8), c = (i % (DT / 8)) * 8;
    uint4 v = z4;
    if (h < hn) {
      const int64_t hr = (int64_t)r * a.n1 + h0 + h;
      v = c < D ? ldg16(qb + hr * D + c) : ldg16(qrb + hr * a.dr + (c - D));
    }
    *reinterpret_cast<uint4*>(&Qs[h * QP + c]) = v;
  }
  if (tid < SBH) {
    float m = 0.f, il = 0.f;
    if (tid < hn) {
      const int64_t hr = (int64_t)r * a.n1 + h0 + tid;
      m = a.sm_max[hr];
      il = 1.f / (a.sm_sum[hr] + SEPS);
    }
    s_m[tid] = m * SLOG2E;
    s_il[tid] = il;
  }
  const int32_t* ids = a.sidx ? a.sidx + (int64_t)r * a.topk : nullptr;
  const float sl2 = a.scale * SLOG2E, inv_n1 = 1.f / a.n1;
  for (int t0 = 0; t0 < n; t0 += SBT) {
    const int nv = n - t0 < SBT ? n - t0 : SBT;
    for (int i = tid; i < SBT * (DT / 8); i += SWV * 64) {
      const int t = i / (DT / 8), c = (i % (DT / 8)) * 8;
      uint4 v = z4;
      if (t < nv) {
        const int64_t kr = (int64_t)b * a.s2 + slot_key(a, ids, t0 + t);
        v = c < D ? ldg16(kb + kr * D + c) : ldg16(krb + kr * a.dr + (c - D));
      }
      *reinterpret_cast<uint4*>(&Ks[t * QP + c]) = v;
    }
    __syncthreads();
    {
      constexpr int NKS = KS / SWV;
      const uint16_t* arow = Ks + (lane & 31) * QP + (lane >> 5) * 8 + wave * NKS * 16;
      const uint16_t* brow = Qs + (lane & 31) * QP + (lane >> 5) * 8 + wave * NKS * 16;
      f32x16 s = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks)
        s = Mfma<IO>::m32(*reinterpret_cast<const uint4*>(arow + ks * 16),
                          *reinterpret_cast<const uint4*>(brow + ks * 16), s);
#pragma unroll
      for (int i = 0; i < 16; ++i) part[wave][i][lane] = s[i];
    }
    __syncthreads();
    // element (i, lane): token m32_row(i, lane), head lane % 32; the block's
    // probabilities summed over its heads (the 32 lanes of a half-wave)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = wave * 4 + j;
      const int tk = m32_row(i, lane), h = lane & 31;
      const float sv = part[0][i][lane] + part[1][i][lane] + part[2][i][lane] + part[3][i][lane];
      float pr = h < hn ? __builtin_amdgcn_exp2f(sv * sl2 - s_m[h]) * s_il[h] : 0.f;
#pragma unroll
      for (int o = 16; o >= 1; o >>= 1) pr += __shfl_xor(pr, o, 32);
      if ((lane & 31) == 0 && tk < nv) unsafeAtomicAdd(a.p + (int64_t)r * a.topk + t0 + tk, pr * inv_n1);
    }
    __syncthreads();   // the next tile overwrites Ks and part
  }
}

// Dense teacher over grouped key heads on MFMA: work-group (32 query rows of one batch,
// NKT x 32 keys), one wave per 32-key tile. For each attention head h (key head h / G)
// the rows' q_h and the tiles of key head h / G sit in LDS; S^T[key, row] comes from
// 32x32x16 MFMAs (keys as M) and exp(score - max) / (sum + eps) accumulates over the
// heads in registers, so every p[row, key] is written once, without atomics.
template <int IO, int DT, int NKT>
__global__ __launch_bounds__(NKT * 64) void sli_teacher_heads_kernel(SliArgs a) {
  constexpr int QP = DT + 8;
  constexpr int KS = DT / 16;
  constexpr int NT = NKT * 64;
  __shared__ __attribute__((aligned(16))) uint16_t Qs[32 * QP];
  __shared__ __attribute__((aligned(16))) uint16_t Ks[NKT * 32 * QP];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // XCD-aware order: work-group L runs on XCD L % 8, so XCD x takes the contiguous
  // range [x C, x C + C) of the key-block-major order (C = gridDim.x / 8): the row blocks
  // that share a key block run on one XCD and read its key tiles through one L2
  const int nrb = (a.s1 + 31) / 32, nx = a.batch * nrb;
  const int cpx = gridDim.x / 8;
  const int mo = (int)(blockIdx.x % 8) * cpx + (int)(blockIdx.x / 8);
  if (mo >= nx * ((a.s2 + NKT * 32 - 1) / (NKT * 32))) return;
  const int rbk = mo % nx;
  const int b = rbk / nrb, s0 = (rbk - b * nrb) * 32;
  const int t0 = (mo / nx) * (NKT * 32);
  const int aq = a.act_q[b], ak = a.act_k[b];
  auto slots = [&](int s1) {
    if (s1 >= a.s1 || s1 >= aq) return 0;
    int n = ak - aq + s1 + 1;
    n = n < 0 ? 0 : n;
    return n < a.topk ? n : a.topk;
  };
  // n grows with s1 up to act_q - 1: the block's widest row bounds the keys it sees
  int last = s0 + 31 < a.s1 ? s0 + 31 : a.s1 - 1;
  last = last < aq - 1 ? last : aq - 1;
  if (last < s0 || t0 >= slots(last)) return;
  const int G = a.n1 / a.n2, D = a.d;
  const uint16_t* qb = reinterpret_cast<const uint16_t*>(a.q);
  const uint16_t* qrb = reinterpret_cast<const uint16_t*>(a.qr);
  const uint16_t* kb = reinterpret_cast<const uint16_t*>(a.k);
  const uint16_t* krb = reinterpret_cast<const uint16_t*>(a.kr);
  const uint4 z4 = make_uint4(0, 0, 0, 0);
  const int my_s1 = s0 + (lane & 31);
  const int my_n = slots(my_s1);
  const int64_t my_r = (int64_t)b * a.s1 + my_s1;
  const float sl2 = a.scale * SLOG2E;
  f32x16 pacc;
#pragma unroll
  for (int e = 0; e < 16; ++e) pacc[e] = 0.f;
  // Head h + 1's q rows (and key rows, when its key head changes) are loaded into
  // registers while head h computes (PF: when they fit in 16 chunks per thread; wider
  // rows load in place); LDS-only barriers, so the loads in flight are not drained by
  // them (a full __syncthreads() would wait for them).
  constexpr int QL = (32 * (DT / 8) + NT - 1) / NT, KL = (NKT * 32 * (DT / 8) + NT - 1) / NT;
  constexpr bool PF = QL + KL <= 16;
  uint4 qst[PF ? QL : 1], kst[PF ? KL : 1];
  auto stage = [&](int h) {
    const int kvh = h / G, g = h - kvh * G;
#pragma unroll
    for (int j = 0; j < QL; ++j) {
      const int i = tid + j * NT;
      const int rr = i / (DT / 8), c = (i % (DT / 8)) * 8;
      uint4 v = z4;
      if (i < 32 * (DT / 8) && s0 + rr < a.s1) {
        const int64_t hr = ((int64_t)b * a.s1 + s0 + rr) * a.n1 + h;
        v = c < D ? ldg16(qb + hr * D + c) : ldg16(qrb + hr * a.dr + (c - D));
      }
      qst[j] = v;
    }
    if (g == 0)
#pragma unroll
      for (int j = 0; j < KL; ++j) {
        const int i = tid + j * NT;
        const int jr = i / (DT / 8), c = (i % (DT / 8)) * 8;
        uint4 v = z4;
        if (i < NKT * 32 * (DT / 8) && t0 + jr < a.s2) {
          const int64_t kr = ((int64_t)b * a.s2 + t0 + jr) * a.n2 + kvh;
          v = c < D ? ldg16(kb + kr * D + c) : ldg16(krb + kr * a.dr + (c - D));
        }
        kst[j] = v;
      }
  };
  if constexpr (PF) stage(0);
  for (int h = 0; h < a.n1; ++h) {
    const int kvh = h / G, g = h - kvh * G;
    lds_barrier();   // the previous head's MFMAs are done with Qs / Ks
    if constexpr (PF) {
#pragma unroll
      for (int j = 0; j < QL; ++j) {
        const int i = tid + j * NT;
        if (i < 32 * (DT / 8)) *reinterpret_cast<uint4*>(&Qs[(i / (DT / 8)) * QP + (i % (DT / 8)) * 8]) = qst[j];
      }
      if (g == 0)
#pragma unroll
        for (int j = 0; j < KL; ++j) {
          const int i = tid + j * NT;
          if (i < NKT * 32 * (DT / 8))
            *reinterpret_cast<uint4*>(&Ks[(i / (DT / 8)) * QP + (i % (DT / 8)) * 8]) = kst[j];
        }
    } else {
      for (int i = tid; i < 32 * (DT / 8); i += NT) {
        const int rr = i / (DT / 8), c = (i % (DT / 8)) * 8;
        uint4 v = z4;
        if (s0 + rr < a.s1) {
          const int64_t hr = ((int64_t)b * a.s1 + s0 + rr) * a.n1 + h;
          v = c < D ? ldg16(qb + hr * D + c) : ldg16(qrb + hr * a.dr + (c - D));
        }
        *reinterpret_cast<uint4*>(&Qs[rr * QP + c]) = v;
      }
      if (g == 0)
        for (int i = tid; i < NKT * 32 * (DT / 8); i += NT) {
          const int j = i / (DT / 8), c = (i % (DT / 8)) * 8;
          uint4 v = z4;
          if (t0 + j < a.s2) {
            const int64_t kr = ((int64_t)b * a.s2 + t0 + j) * a.n2 + kvh;
            v = c < D ? ldg16(kb + kr * D + c) : ldg16(krb + kr * a.dr + (c - D));
          }
          *reinterpret_cast<uint4*>(&Ks[j * QP + c]) = v;
        }
    }
    // this head's statistics are requested before the next head's rows (loads retire
    // in order, so waiting for them does not wait for the prefetch)
    float m = 0.f, il = 0.f;
    if (my_n > 0) {
      const int64_t si = (((int64_t)b * a.n2 + kvh) * a.s1 + my_s1) * G + g;
      m = a.sm_max[si] * SLOG2E;
      il = a.sm_sum[si];
    }
    if constexpr (PF)
      if (h + 1 < a.n1) stage(h + 1);
    il = my_n > 0 ? 1.f / (il + SEPS) : 0.f;
    lds_barrier();
    const uint16_t* arow = Ks + (wave * 32 + (lane & 31)) * QP + (lane >> 5) * 8;
    const uint16_t* brow = Qs + (lane & 31) * QP + (lane >> 5) * 8;
    f32x16 sc = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      sc = Mfma<IO>::m32(*reinterpret_cast<const uint4*>(arow + ks * 16),
                         *reinterpret_cast<const uint4*>(brow + ks * 16), sc);
#pragma unroll
    for (int e = 0; e < 16; ++e) pacc[e] += __builtin_amdgcn_exp2f(sc[e] * sl2 - m) * il;
  }
  const float inv_n1 = 1.f / a.n1;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int t = t0 + wave * 32 + m32_row(e, lane);
    if (t < my_n) a.p[my_r * a.topk + t] = pacc[e] * inv_n1;
  }
}

// ---------------------------------------------------------------- student
// MFMA operand whose K runs down the rows of a row-major 16-bit LDS array X: lane l
// receives X[k0 + 8 (l / 32) + j][c0 + l % 32], j = 0..7 (two transposed reads).
__device__ __forceinline__ uint4 s_tr_frag(const uint16_t* X, int pitch, int c0, int k0, int lane) {
  const int g16 = lane >> 4, c16 = lane & 15;
  const int col = c0 + (g16 & 1) * 16 + 4 * (c16 & 3);
  const int k = k0 + (g16 >> 1) * 8 + (c16 >> 2);
  const uint2 lo = ds_read_tr(X + k * pitch + col);
  const uint2 hi = ds_read_tr(X + (k + 4) * pitch + col);
  return make_uint4(lo.x, lo.y, hi.x, hi.y);
}

// One work-group (4 waves) per row. The row's qi block is taken in NHH passes of GP =
// 32 NGB heads (NHH = 2 when the whole block would not fit LDS: Nidx1 > 64 at D_idx = 512);
// wave w < NGB owns heads 32w..32w+31 of a pass. Per tile of 32 slots, dot^T[slot, head] =
// ki qi^T on 32x32x16 MFMAs (slots as M), and relu * w summed over the heads (half-wave
// shuffles, then across waves and passes) is I. The first sweep over the tiles keeps a
// running max / sum of I (the softmax statistics: the LSE-only mode stops there) and
// stores I per slot, in LDS or, for rows of more than SLI_MAX_SLOTS slots (BIG), in a
// workspace row. The second sweep recomputes the dots and gives dW (per lane), ds = dI w
// [relu > 0] (to LDS as [head][slot], split in two io-dtype parts), dQI[head, col] += ds ki
// (registers) and dKI[slot, col] = ds^T qi, added at the slot's key row with fp32 atomics.
template <int IO, int DI, int NGB, int NHH, bool BIG>
__global__ __launch_bounds__(256) void sli_student_kernel(SliArgs a) {
  constexpr int GP = 32 * NGB;         // heads of one pass, padded to whole blocks
  constexpr int QIP = DI + 8;          // qi / ki row pitch: odd count of 16-byte units
  constexpr int DP = SBT + 8;          // ds row pitch
  constexpr int KS = DI / 16;          // k-steps of the dots
  constexpr int NCB = DI / 32;         // 32-column blocks of dQI / dKI
  constexpr int JK = (NCB + SWV - 1) / SWV;   // dKI column blocks per wave, at most
  __shared__ __attribute__((aligned(16))) uint16_t QIs[GP * QIP];
  __shared__ __attribute__((aligned(16))) uint16_t KIs[SBT * QIP];
  // ds = hi + lo, both in the io dtype (hi = ds rounded, lo = the rounding error
  // rounded): the products use both, so ds keeps ~22 bits through the MFMAs -- the
  // indexer softmax is sharply peaked, ds reaches |w|, and one 16-bit rounding of it
  // alone would cost ~2^-11 relative on d_key_index
  __shared__ __attribute__((aligned(16))) uint16_t dSs[2][GP * DP];
  __shared__ float s_i_lds[BIG ? 1 : SLI_MAX_SLOTS];  // I, then dI (BIG: a workspace row instead)
  __shared__ float s_w[GP];
  __shared__ float red[SWV][SBT];
  __shared__ float s_red[SWV];
  __shared__ int s_tok[SBT];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = blockIdx.x;
  int b, s1;
  const int n = row_slots(a, r, b, s1);
  const int G = a.nidx1;
  uint16_t* dqio = reinterpret_cast<uint16_t*>(a.dqi);
  const int64_t qrow = (int64_t)r * G;
  auto store_w = [&](int g, float v) {
    if (a.wdt == DSA_DTYPE_F32) reinterpret_cast<float*>(a.dw)[qrow + g] = v;
    else if (a.wdt == DSA_DTYPE_BF16) reinterpret_cast<uint16_t*>(a.dw)[qrow + g] = f32_to_bf16_rne(v);
    else reinterpret_cast<uint16_t*>(a.dw)[qrow + g] = f32_to_f16_rne(v);
  };
  const bool lse_only = a.lse_max != nullptr;
  if (lse_only && n == 0) {
    if (tid == 0) { a.lse_max[r] = -INFINITY; a.lse_sum[r] = 0.f; }
    return;
  }
  // no slot, or (dense, given stats) an empty indexer softmax: zero gradients, zero loss
  if (n == 0 || (a.isum && !(a.isum[r] > 0.f))) {
    for (int i = tid; i < G * DI; i += 256) dqio[qrow * DI + i] = 0;
    for (int g = tid; g < G; g += 256) store_w(g, 0.f);
    if (tid == 0) a.row_loss[r] = 0.f;
    return;
  }
  float* s_i = BIG ? a.ibuf + (int64_t)r * a.topk : s_i_lds;
  const uint16_t* qib = reinterpret_cast<const uint16_t*>(a.qi);
  const uint16_t* kib = reinterpret_cast<const uint16_t*>(a.ki);
  const uint4 z4 = make_uint4(0, 0, 0, 0);
  // qi rows and weights of pass hh: heads hh GP .. hh GP + GP - 1 (zero past Nidx1)
  auto load_qi = [&](int hh) {
    for (int i = tid; i < GP * (DI / 8); i += 256) {
      const int g = i / (DI / 8), c = (i % (DI / 8)) * 8, gg = hh * GP + g;
      *reinterpret_cast<uint4*>(&QIs[g * QIP + c]) = ldg16_or0(gg < G, qib + (qrow + gg) * DI + c);
    }
    for (int g = tid; g < GP; g += 256) s_w[g] = hh * GP + g < G ? ld_w(a.w, a.wdt, qrow + hh * GP + g) : 0.f;
  };
  const int32_t* ids = a.sidx ? a.sidx + (int64_t)r * a.topk : nullptr;

  // ki rows of a tile are fetched into registers one tile ahead (in flight while the
  // current tile computes) and committed to LDS once every wave is done with it
  constexpr int LPT = SBT * (DI / 8) / 256;   // 16-byte chunks per thread per tile
  uint4 stage[LPT];
  int stok = -1;
  auto fetch_tile = [&](int t0) {
    const int nv = n - t0 < SBT ? n - t0 : SBT;
#pragma unroll
    for (int j = 0; j < LPT; ++j) {
      const int i = tid + j * 256;
      const int t = i / (DI / 8), c = (i % (DI / 8)) * 8;
      stage[j] = ldg16_or0(t < nv, kib + ((int64_t)b * a.s2 + slot_key(a, ids, t0 + (t < nv ? t : 0))) * DI + c);
    }
    if (tid < SBT) stok = tid < nv ? b * a.s2 + slot_key(a, ids, t0 + tid) : -1;
  };
  auto commit_tile = [&]() {
#pragma unroll
    for (int j = 0; j < LPT; ++j) {
      const int i = tid + j * 256;
      const int t = i / (DI / 8), c = (i % (DI / 8)) * 8;
      *reinterpret_cast<uint4*>(&KIs[t * QIP + c]) = stage[j];
    }
    if (tid < SBT) s_tok[tid] = stok;
  };
  // dot^T of this wave's head block over the tile: element e -> slot m32_row(e, lane),
  // head 32 wave + lane % 32 (of the current pass)
  auto dots = [&]() -> f32x16 {
    f32x16 acc = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    const uint16_t* arow = KIs + (lane & 31) * QIP + (lane >> 5) * 8;
    const uint16_t* brow = QIs + (32 * wave + (lane & 31)) * QIP + (lane >> 5) * 8;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      acc = Mfma<IO>::m32(*reinterpret_cast<const uint4*>(arow + ks * 16),
                          *reinterpret_cast<const uint4*>(brow + ks * 16), acc);
    return acc;
  };
  if (NHH == 1) load_qi(0);   // one pass: the block stays for both sweeps

  // ---- first sweep: I per slot, with a running max / sum (wave 0, lanes < 32)
  float run_m = -INFINITY, run_l = 0.f;
  fetch_tile(0);
  for (int t0 = 0; t0 < n; t0 += SBT) {
    const int nv = n - t0 < SBT ? n - t0 : SBT;
    commit_tile();   // the previous tile's readers are behind the last barrier
    if (t0 + SBT < n) fetch_tile(t0 + SBT);
    float iv = 0.f;   // thread tid < nv: I of slot t0 + tid, summed over the passes
#pragma unroll
    for (int hh = 0; hh < NHH; ++hh) {
      if (NHH > 1) load_qi(hh);
      __syncthreads();
      if (wave < NGB) {
        const f32x16 acc = dots();
        const float wg = s_w[32 * wave + (lane & 31)];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          float v = wg * fmaxf(acc[e], 0.f);
#pragma unroll
          for (int o = 16; o >= 1; o >>= 1) v += __shfl_xor(v, o, 32);
          if ((lane & 31) == 0) red[wave][m32_row(e, lane)] = v;
        }
      }
      __syncthreads();
      if (tid < nv) {
#pragma unroll
        for (int w = 0; w < NGB; ++w) iv += red[w][tid];
      }
    }
    if (tid < SBT) {
      const float v = tid < nv ? iv : -INFINITY;
      if (!lse_only && tid < nv) s_i[t0 + tid] = v;
      float tm = v;
#pragma unroll
      for (int o = 16; o >= 1; o >>= 1) tm = fmaxf(tm, __shfl_xor(tm, o, 32));
      const float nm = fmaxf(run_m, tm);   // finite: a tile holds at least one slot
      float e = tid < nv ? expf(v - nm) : 0.f;
#pragma unroll
      for (int o = 16; o >= 1; o >>= 1) e += __shfl_xor(e, o, 32);
      run_l = run_l * expf(run_m - nm) + e;   // the first tile: exp(-inf) = 0
      run_m = nm;
    }
    // the next tile overwrites KIs and s_tok: every wave's dots and the reads of red
    // are behind the barrier above or in program order before the next one
  }
  // ---- softmax of I over the n slots, dI = sI - p, the row's loss
  auto block_sum = [&](float v) {
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    if (lane == 0) s_red[wave] = v;
    __syncthreads();
    const float t = s_red[0] + s_red[1] + s_red[2] + s_red[3];
    __syncthreads();
    return t;
  };
  // sparse: sI = e / (sum e + eps); dense: sI = e / max(sum e, eps), with the given
  // stats when the caller has them
  float mx, inv;
  if (a.isum) {
    mx = a.imax[r];
    inv = 1.f / fmaxf(a.isum[r], SEPS);
  } else {
    if (tid == 0) {
      s_red[0] = run_m;
      s_red[1] = run_l;
    }
    __syncthreads();
    mx = s_red[0];
    const float es = s_red[1];
    __syncthreads();
    if (lse_only) {
      if (tid == 0) { a.lse_max[r] = mx; a.lse_sum[r] = es; }
      return;
    }
    inv = ids ? 1.f / (es + SEPS) : 1.f / fmaxf(es, SEPS);
  }
  __syncthreads();   // every I stored (BIG: in the workspace row) before it is read back
  float ls = 0.f;
  for (int k = tid; k < n; k += 256) {
    const float sv = expf(s_i[k] - mx) * inv;
    const float pv = a.p[(int64_t)r * a.topk + k];
    const float pc = fmaxf(pv, SEPS), sc = fmaxf(sv, SEPS);
    ls += pc * (logf(pc) - logf(sc));
    s_i[k] = sv - pv;   // dI
  }
  const float row_loss = block_sum(ls);
  if (tid == 0) a.row_loss[r] = row_loss;

  // ---- second sweep, per pass of GP heads
#pragma unroll 1
  for (int hh = 0; hh < NHH; ++hh) {
    if (NHH > 1) {
      __syncthreads();   // the previous pass is done with QIs, s_w and dSs
      load_qi(hh);
    }
    f32x16 dq[NCB];
#pragma unroll
    for (int j = 0; j < NCB; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) dq[j][e] = 0.f;
    float dwl = 0.f;
    fetch_tile(0);
    for (int t0 = 0; t0 < n; t0 += SBT) {
      const int nv = n - t0 < SBT ? n - t0 : SBT;
      commit_tile();
      if (t0 + SBT < n) fetch_tile(t0 + SBT);
      __syncthreads();
      if (wave < NGB) {
        const f32x16 acc = dots();
        const int g = 32 * wave + (lane & 31);
        const float wg = s_w[g];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int tk = m32_row(e, lane);
          const float di = tk < nv ? s_i[t0 + tk] : 0.f;
          dwl += fmaxf(acc[e], 0.f) * di;
          const float ds = acc[e] > 0.f ? di * wg : 0.f;
          const uint16_t hi = from_f32<IO>(ds);
          dSs[0][g * DP + tk] = hi;
          dSs[1][g * DP + tk] = from_f32<IO>(ds - to_f32<IO>(hi));
        }
      }
      __syncthreads();
      // dQI[head, col] += ds[head, slot] ki[slot, col]   (this wave's head block)
      if (wave < NGB) {
#pragma unroll
        for (int kq = 0; kq < SBT / 16; ++kq) {
          const int off = (32 * wave + (lane & 31)) * DP + kq * 16 + (lane >> 5) * 8;
          const uint4 ah = *reinterpret_cast<const uint4*>(dSs[0] + off);
          const uint4 al = *reinterpret_cast<const uint4*>(dSs[1] + off);
#pragma unroll
          for (int j = 0; j < NCB; ++j) {
            const uint4 bv = s_tr_frag(KIs, QIP, 32 * j, kq * 16, lane);
            dq[j] = Mfma<IO>::m32(ah, bv, dq[j]);
            dq[j] = Mfma<IO>::m32(al, bv, dq[j]);
          }
        }
      }
      // dKI[slot, col] = ds^T qi over the pass's heads, this wave's column blocks
#pragma unroll
      for (int jj = 0; jj < JK; ++jj) {
        const int j = wave + SWV * jj;
        if (j < NCB) {
          f32x16 c = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kq = 0; kq < GP / 16; ++kq) {
            const uint4 bv = s_tr_frag(QIs, QIP, 32 * j, kq * 16, lane);
            c = Mfma<IO>::m32(s_tr_frag(dSs[0], DP, 0, kq * 16, lane), bv, c);
            c = Mfma<IO>::m32(s_tr_frag(dSs[1], DP, 0, kq * 16, lane), bv, c);
          }
          float* dst = a.dki_acc + 32 * j + (lane & 31);
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int kr = s_tok[m32_row(e, lane)];
            if (kr >= 0) unsafeAtomicAdd(dst + (int64_t)kr * DI, c[e]);
          }
        }
      }
      __syncthreads();   // the next tile overwrites KIs, dSs and s_tok
    }
    // ---- dQI of the pass (element e -> head hh GP + 32 wave + m32_row(e, lane), column
    // 32 j + lane % 32) and dW
    if (wave < NGB) {
#pragma unroll
      for (int j = 0; j < NCB; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int g = hh * GP + 32 * wave + m32_row(e, lane);
          if (g < G) dqio[(qrow + g) * DI + 32 * j + (lane & 31)] = from_f32<IO>(dq[j][e]);
        }
      const float v = dwl + __shfl_xor(dwl, 32);   // the two slot halves of head lane % 32
      const int g = hh * GP + 32 * wave + lane;
      if (lane < 32 && g < G) store_w(g, v);
    }
  }
}

// Wave-per-tile student for D_idx = 128, Nidx1 <= 32 MT and rows of at most
// SLI_MAX_SLOTS slots. One work-group (4 waves) per row; wave w takes the 32-slot
// tiles w, w + 4, ... of both sweeps, so no block barrier is needed per tile. Heads
// are the MFMA M dimension (dots[head, slot] = qi ki^T, the row's qi fragments in
// VGPRs): a lane holds 16 heads of one slot, and I = sum_g w[g] relu(dots) is an
// in-lane sum plus one lane-half swap. A wave stages its tile's ki rows in a private
// LDS tile (fetched one tile ahead into registers) and writes the tile's ds (hi and
// lo parts, as in sli_student_kernel) to a private [slot][head] LDS tile; from there
// dQI[head, col] += ds ki is accumulated in registers over the wave's tiles (the
// four partials are added once per row, in wave order) and dKI[slot, col] = ds^T qi
// is added at the slot's key row with fp32 atomics.
template <int IO, int MT, bool KM>
__global__ __launch_bounds__(256) void sli_student_wt_kernel(SliArgs a) {
  constexpr int DI = 128;
  constexpr int GP = 32 * MT;          // heads, padded to whole blocks
  constexpr int QIP = DI + 8;          // qi / ki row pitch: odd count of 16-byte units
  constexpr int DSP = GP + 8;          // ds tile row pitch ([slot][head])
  constexpr int KK = DI / 16;          // k-steps of the dots
  constexpr int NCB = DI / 32;         // 32-column blocks of dQI / dKI
  constexpr int NW = 4;                // waves
  constexpr int LPW = SBT * (DI / 8) / 64;   // 16-byte ki chunks per lane per tile
  static_assert(NW * SBT * QIP * 2 >= GP * DI * 4, "the dQI sum fits the ki tiles");
  __shared__ __attribute__((aligned(16))) uint16_t QIs[GP * QIP];
  __shared__ __attribute__((aligned(16))) uint16_t KIw[NW][SBT * QIP];
  __shared__ __attribute__((aligned(16))) uint16_t dSw[NW][2][SBT * DSP];
  __shared__ __attribute__((aligned(16))) float s_i[SLI_MAX_SLOTS];   // I, then dI
  __shared__ float s_w[GP];
  __shared__ float s_st[NW][2];          // the waves' running max / sum of I
  __shared__ float s_red[NW];
  __shared__ float s_dw[NW][GP];
  __shared__ int s_key[NW][SBT];         // key row of each slot of the wave's tile (-1: none)

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = blockIdx.x;
  int b, s1;
  const int n = row_slots(a, r, b, s1);
  const int G = a.nidx1;
  uint16_t* dqio = reinterpret_cast<uint16_t*>(a.dqi);
  const int64_t qrow = (int64_t)r * G;
  auto store_w = [&](int g, float v) {
    if (a.wdt == DSA_DTYPE_F32) reinterpret_cast<float*>(a.dw)[qrow + g] = v;
    else if (a.wdt == DSA_DTYPE_BF16) reinterpret_cast<uint16_t*>(a.dw)[qrow + g] = f32_to_bf16_rne(v);
    else reinterpret_cast<uint16_t*>(a.dw)[qrow + g] = f32_to_f16_rne(v);
  };
  const bool lse_only = a.lse_max != nullptr;
  if (lse_only && n == 0) {
    if (tid == 0) { a.lse_max[r] = -INFINITY; a.lse_sum[r] = 0.f; }
    return;
  }
  if (n == 0 || (a.isum && !(a.isum[r] > 0.f))) {
    for (int i = tid; i < G * DI; i += 256) dqio[qrow * DI + i] = 0;
    for (int g = tid; g < G; g += 256) store_w(g, 0.f);
    if (tid == 0) a.row_loss[r] = 0.f;
    return;
  }
  const uint16_t* qib = reinterpret_cast<const uint16_t*>(a.qi);
  const uint16_t* kib = reinterpret_cast<const uint16_t*>(a.ki);
  const uint4 z4 = make_uint4(0, 0, 0, 0);
  // the qi block and weights (zero past Nidx1): to LDS for dKI, and the dots' A
  // fragments (head 32 mt + lane % 32, k = 16 kk + 8 (lane / 32) ..) to VGPRs
  for (int i = tid; i < GP * (DI / 8); i += 256) {
    const int g = i / (DI / 8), c = (i % (DI / 8)) * 8;
    *reinterpret_cast<uint4*>(&QIs[g * QIP + c]) = ldg16_or0(g < G, qib + (qrow + g) * DI + c);
  }
  for (int g = tid; g < GP; g += 256) s_w[g] = g < G ? ld_w(a.w, a.wdt, qrow + g) : 0.f;
  uint4 qf[MT][KK];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const int g = 32 * mt + (lane & 31);
      qf[mt][kk] = ldg16_or0(g < G, qib + (qrow + g) * DI + kk * 16 + (lane >> 5) * 8);
    }
  __syncthreads();
  float wv[MT][16];   // weight of head 32 mt + m32_row(e, lane)
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int e = 0; e < 16; ++e) wv[mt][e] = s_w[32 * mt + m32_row(e, lane)];
  const int32_t* ids = a.sidx ? a.sidx + (int64_t)r * a.topk : nullptr;
  const int ntiles = (n + SBT - 1) / SBT;
  uint16_t* const kt = KIw[wave];
  uint16_t* const dsh = dSw[wave][0];
  uint16_t* const dsl = dSw[wave][1];

  // sparse mode: the ids of the next tile to fetch (slot lane % 32), loaded one tile
  // ahead so that a fetch never waits for an id load
  int idn = 0;
  auto load_ids = [&](int t) {
    const int sl = t * SBT + (lane & 31);
    if (ids) idn = sl < n ? ids[sl] : 0;
  };
  // ki rows of tile t: lane l holds chunks l + 64 j of the 32 x DI tile
  uint4 stg[LPW];
  int skey = -1;
  auto fetch = [&](int t) {
    const int t0 = t * SBT, nv = n - t0 < SBT ? n - t0 : SBT;
#pragma unroll
    for (int j = 0; j < LPW; ++j) {
      const int i = lane + 64 * j;
      const int row = i / (DI / 8), c = (i % (DI / 8)) * 8;
      const int key = ids ? clip_id(__shfl(idn, row), a.s2) : t0 + row;
      stg[j] = ldg16_or0(row < nv, kib + ((int64_t)b * a.s2 + key) * DI + c);
    }
    if (lane < SBT) skey = lane < nv ? b * a.s2 + (ids ? clip_id(idn, a.s2) : t0 + lane) : -1;
  };
  auto first_fetch = [&]() {
    if (wave < ntiles) {
      load_ids(wave);
      fetch(wave);
      load_ids(wave + NW);
    }
  };
  auto next_fetch = [&](int t) {
    if (t + NW < ntiles) {
      fetch(t + NW);
      load_ids(t + 2 * NW);
    }
  };
  // this wave's reads of its previous tile are complete (LDS runs a wave's accesses in order)
  auto commit = [&]() {
#pragma unroll
    for (int j = 0; j < LPW; ++j) {
      const int i = lane + 64 * j;
      *reinterpret_cast<uint4*>(&kt[(i / (DI / 8)) * QIP + (i % (DI / 8)) * 8]) = stg[j];
    }
    if (lane < SBT) s_key[wave][lane] = skey;
  };
  // dots of the tile in kt: acc[mt] element e -> head 32 mt + m32_row(e, lane), slot lane % 32
  auto dots = [&](f32x16 (&acc)[MT]) {
    uint4 bk[KK];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
      bk[kk] = *reinterpret_cast<const uint4*>(kt + (lane & 31) * QIP + kk * 16 + (lane >> 5) * 8);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[mt][i] = 0.f;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt] = Mfma<IO>::m32(qf[mt][kk], bk[kk], acc[mt]);
  };
  auto max32 = [](float v) {
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 32));
    return v;
  };
  auto sum32 = [](float v) {
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) v += __shfl_xor(v, o, 32);
    return v;
  };

  // ---- first sweep: I per slot, with this wave's running max / sum
  float run_m = -INFINITY, run_l = 0.f;
  first_fetch();
  for (int t = wave; t < ntiles; t += NW) {
    commit();
    next_fetch(t);
    f32x16 acc[MT];
    dots(acc);
    float p4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int e = 0; e < 16; ++e) p4[e & 3] += fmaxf(acc[mt][e], 0.f) * wv[mt][e];
    const float iv = add_half_swap((p4[0] + p4[1]) + (p4[2] + p4[3]));   // slot lane % 32, both halves
    const int t0 = t * SBT, nv = n - t0 < SBT ? n - t0 : SBT, slot = lane & 31;
    const bool ok = slot < nv;
    if (!lse_only && lane < 32 && ok) s_i[t0 + slot] = iv;
    const float nm = fmaxf(run_m, max32(ok ? iv : -INFINITY));   // finite: the tile holds a slot
    const float ex = sum32(ok ? expf(iv - nm) : 0.f);
    run_l = run_l * expf(run_m - nm) + ex;   // the first tile: exp(-inf) = 0
    run_m = nm;
  }
  if (lane == 0) {
    s_st[wave][0] = run_m;
    s_st[wave][1] = run_l;
  }
  auto block_sum = [&](float v) {
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    if (lane == 0) s_red[wave] = v;
    __syncthreads();
    const float t = s_red[0] + s_red[1] + s_red[2] + s_red[3];
    __syncthreads();
    return t;
  };
  __syncthreads();   // the waves' statistics and every I
  float mx, inv;
  if (a.isum) {
    mx = a.imax[r];
    inv = 1.f / fmaxf(a.isum[r], SEPS);
  } else {
    float m = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) m = fmaxf(m, s_st[w][0]);
    float es = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w)
      if (s_st[w][0] > -INFINITY) es += s_st[w][1] * expf(s_st[w][0] - m);
    mx = m;
    if (lse_only) {
      if (tid == 0) { a.lse_max[r] = mx; a.lse_sum[r] = es; }
      return;
    }
    inv = ids ? 1.f / (es + SEPS) : 1.f / fmaxf(es, SEPS);
  }
  float ls = 0.f;
  for (int k = tid; k < n; k += 256) {
    const float sv = expf(s_i[k] - mx) * inv;
    const float pv = a.p[(int64_t)r * a.topk + k];
    const float pc = fmaxf(pv, SEPS), sc = fmaxf(sv, SEPS);
    ls += pc * (logf(pc) - logf(sc));
    s_i[k] = sv - pv;   // dI
    if constexpr (KM) {   // for the key-major dKI pass
      if (ids) unsafeAtomicAdd(a.dib + (int64_t)r * a.dib_ld + slot_key(a, ids, k), sv - pv);
      else a.p[(int64_t)r * a.topk + k] = sv - pv;
    }
  }
  const float row_loss = block_sum(ls);   // its barriers also publish every dI
  if (tid == 0) a.row_loss[r] = row_loss;
  // KM: dI of slot pairs (2m, 2m + 1) as packed hi and lo parts in the io dtype (the
  // ds tiles' LDS, unused in this mode), and dI = 0 past the row's slots up to the
  // last tile's end
  uint32_t* const s_dih = reinterpret_cast<uint32_t*>(&dSw[0][0][0]);
  uint32_t* const s_dil = s_dih + SLI_MAX_SLOTS / 2;
  if constexpr (KM) {
    static_assert(sizeof(dSw) >= SLI_MAX_SLOTS * 4, "the dI pairs fit the ds tiles");
    for (int m = tid; m < ntiles * (SBT / 2); m += 256) {
      const float d0 = 2 * m < n ? s_i[2 * m] : 0.f, d1 = 2 * m + 1 < n ? s_i[2 * m + 1] : 0.f;
      const uint16_t h0 = from_f32<IO>(d0), h1 = from_f32<IO>(d1);
      const uint16_t l0 = from_f32<IO>(d0 - to_f32<IO>(h0)), l1 = from_f32<IO>(d1 - to_f32<IO>(h1));
      s_dih[m] = h0 | ((uint32_t)h1 << 16);
      s_dil[m] = l0 | ((uint32_t)l1 << 16);
      if (2 * m >= n) s_i[2 * m] = 0.f;
      if (2 * m + 1 >= n) s_i[2 * m + 1] = 0.f;
    }
    __syncthreads();
  }

  // ---- second sweep
  f32x16 dq[MT][NCB];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < NCB; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) dq[mt][j][e] = 0.f;
  float dwh[MT] = {};   // KM: dW of head 32 mt + lane % 32 over this lane's slots
  if constexpr (KM) {
    // dots with slots as M (acc[mt] element e: slot m32_row(e, lane), head 32 mt +
    // lane % 32). A lane then holds one head and four groups of four consecutive
    // slots, so the dQI operand [head, 8 slots] of k-step kq is the masked dI pairs of
    // groups 2 kq and 2 kq + 1 after one half swap per register pair: no LDS round
    // trip for ds; w is applied to dQI once per row.
    first_fetch();
    for (int t = wave; t < ntiles; t += NW) {
      commit();
      next_fetch(t);
      f32x16 acc[MT];
      {
        uint4 bk[KK];
#pragma unroll
        for (int kk = 0; kk < KK; ++kk)
          bk[kk] = *reinterpret_cast<const uint4*>(kt + (lane & 31) * QIP + kk * 16 + (lane >> 5) * 8);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int i = 0; i < 16; ++i) acc[mt][i] = 0.f;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) acc[mt] = Mfma<IO>::m32(bk[kk], qf[mt][kk], acc[mt]);
      }
      // group g of this lane: slots t0 + 8 g + 4 (lane / 32) + 0 .. 3
      const int sb = t * SBT + 4 * (lane >> 5);
      float dv[16];
      uint32_t hp[8], lp[8];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 f = *reinterpret_cast<const float4*>(&s_i[sb + 8 * g]);
        dv[4 * g] = f.x; dv[4 * g + 1] = f.y; dv[4 * g + 2] = f.z; dv[4 * g + 3] = f.w;
        const uint2 h = *reinterpret_cast<const uint2*>(&s_dih[(sb + 8 * g) / 2]);
        const uint2 l = *reinterpret_cast<const uint2*>(&s_dil[(sb + 8 * g) / 2]);
        hp[2 * g] = h.x; hp[2 * g + 1] = h.y;
        lp[2 * g] = l.x; lp[2 * g + 1] = l.y;
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        float dw = 0.f;
#pragma unroll
        for (int e = 0; e < 16; ++e) dw += fmaxf(acc[mt][e], 0.f) * dv[e];
        dwh[mt] += dw;
#pragma unroll
        for (int kq = 0; kq < SBT / 16; ++kq) {
          uint32_t xh[2], yh[2], xl[2], yl[2];
#pragma unroll
          for (int pp = 0; pp < 2; ++pp) {
            const int ex = 8 * kq + 2 * pp, ey = ex + 4;
            const uint32_t mx = (acc[mt][ex] > 0.f ? 0xFFFFu : 0u) | (acc[mt][ex + 1] > 0.f ? 0xFFFF0000u : 0u);
            const uint32_t my = (acc[mt][ey] > 0.f ? 0xFFFFu : 0u) | (acc[mt][ey + 1] > 0.f ? 0xFFFF0000u : 0u);
            xh[pp] = mx & hp[4 * kq + pp];
            xl[pp] = mx & lp[4 * kq + pp];
            yh[pp] = my & hp[4 * kq + 2 + pp];
            yl[pp] = my & lp[4 * kq + 2 + pp];
          }
          swap_halves(xh[0], yh[0]);
          swap_halves(xh[1], yh[1]);
          swap_halves(xl[0], yl[0]);
          swap_halves(xl[1], yl[1]);
          const uint4 ah = make_uint4(xh[0], xh[1], yh[0], yh[1]), al = make_uint4(xl[0], xl[1], yl[0], yl[1]);
#pragma unroll
          for (int j = 0; j < NCB; ++j) {
            const uint4 bv = s_tr_frag(kt, QIP, 32 * j, kq * 16, lane);
            dq[mt][j] = Mfma<IO>::m32(ah, bv, dq[mt][j]);
            dq[mt][j] = Mfma<IO>::m32(al, bv, dq[mt][j]);
          }
        }
      }
    }
  }
  float dwp[MT][16];   // dW of head 32 mt + m32_row(e, lane) over this lane's slots
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int e = 0; e < 16; ++e) dwp[mt][e] = 0.f;
  if constexpr (!KM) {
  first_fetch();
  for (int t = wave; t < ntiles; t += NW) {
    commit();
    next_fetch(t);
    f32x16 acc[MT];
    dots(acc);
    const int t0 = t * SBT, nv = n - t0 < SBT ? n - t0 : SBT, slot = lane & 31;
    const float di = slot < nv ? s_i[t0 + slot] : 0.f;
    // ds = dI w [dots > 0] to the [slot][head] tile, hi and lo parts; elements
    // 4q .. 4q + 3 are heads 32 mt + 8 q + 4 (lane / 32) + 0 .. 3 (one 8-byte store)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint16_t hi[4], lo[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int e = 4 * q + u;
          const float x = acc[mt][e];
          dwp[mt][e] += fmaxf(x, 0.f) * di;
          const float dsv = x > 0.f ? di * wv[mt][e] : 0.f;
          hi[u] = from_f32<IO>(dsv);
          lo[u] = from_f32<IO>(dsv - to_f32<IO>(hi[u]));
        }
        const int col = 32 * mt + 8 * q + 4 * (lane >> 5);
        *reinterpret_cast<uint2*>(dsh + slot * DSP + col) =
            make_uint2(hi[0] | ((uint32_t)hi[1] << 16), hi[2] | ((uint32_t)hi[3] << 16));
        *reinterpret_cast<uint2*>(dsl + slot * DSP + col) =
            make_uint2(lo[0] | ((uint32_t)lo[1] << 16), lo[2] | ((uint32_t)lo[3] << 16));
      }
    // dQI[head, col] += ds[head, slot] ki[slot, col]
#pragma unroll
    for (int kq = 0; kq < SBT / 16; ++kq) {
      uint4 ah[MT], al[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        ah[mt] = s_tr_frag(dsh, DSP, 32 * mt, kq * 16, lane);
        al[mt] = s_tr_frag(dsl, DSP, 32 * mt, kq * 16, lane);
      }
#pragma unroll
      for (int j = 0; j < NCB; ++j) {
        const uint4 bv = s_tr_frag(kt, QIP, 32 * j, kq * 16, lane);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          dq[mt][j] = Mfma<IO>::m32(ah[mt], bv, dq[mt][j]);
          dq[mt][j] = Mfma<IO>::m32(al[mt], bv, dq[mt][j]);
        }
      }
    }
    // dKI[slot, col] = sum_head ds[head, slot] qi[head, col], added at the slot's key row
    f32x16 c[NCB];
#pragma unroll
    for (int j = 0; j < NCB; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) c[j][e] = 0.f;
#pragma unroll
    for (int kq = 0; kq < GP / 16; ++kq) {
      const int off = (lane & 31) * DSP + kq * 16 + (lane >> 5) * 8;
      const uint4 ah = *reinterpret_cast<const uint4*>(dsh + off);
      const uint4 al = *reinterpret_cast<const uint4*>(dsl + off);
#pragma unroll
      for (int j = 0; j < NCB; ++j) {
        const uint4 bv = s_tr_frag(QIs, QIP, 32 * j, kq * 16, lane);
        c[j] = Mfma<IO>::m32(ah, bv, c[j]);
        c[j] = Mfma<IO>::m32(al, bv, c[j]);
      }
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int kr = s_key[wave][m32_row(e, lane)];
      if (kr >= 0) {
        float* dst = a.dki_acc + (int64_t)kr * DI + (lane & 31);
#pragma unroll
        for (int j = 0; j < NCB; ++j) unsafeAtomicAdd(dst + 32 * j, c[j][e]);
      }
    }
  }
  }
  // ---- dW: each head's sum over this wave's slots (KM: the two lane halves; else
  // the 32 lanes of its half), then over the waves
  if constexpr (KM) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const float v = dwh[mt] + __shfl_xor(dwh[mt], 32);
      if (lane < 32) s_dw[wave][32 * mt + lane] = v;
    }
  } else {
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float v = sum32(dwp[mt][e]);
      if ((lane & 31) == 0) s_dw[wave][32 * mt + m32_row(e, lane)] = v;
    }
  }
  // ---- dQI: the waves' partials added in wave order in LDS (the ki tiles are free)
  float* const qacc = reinterpret_cast<float*>(&KIw[0][0]);   // [GP][DI]
  __syncthreads();
#pragma unroll 1
  for (int w = 0; w < NW; ++w) {
    if (wave == w) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < NCB; ++j)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            float* p = qacc + (32 * mt + m32_row(e, lane)) * DI + 32 * j + (lane & 31);
            const float v = KM ? dq[mt][j][e] * wv[mt][e] : dq[mt][j][e];   // KM: the factored w
            *p = (w == 0 ? 0.f : *p) + v;
          }
    }
    __syncthreads();
  }
  for (int i = tid; i < G * DI; i += 256) dqio[qrow * DI + i] = from_f32<IO>(qacc[i]);
  for (int g = tid; g < G; g += 256) store_w(g, (s_dw[0][g] + s_dw[1][g]) + (s_dw[2][g] + s_dw[3][g]));
}

// Head-split student for the key-major mode and the softmax-LSE mode (D_idx = 128,
// 32 < Nidx1 <= 64, rows of at most SLI_MAX_SLOTS slots). One work-group of 8 waves per
// row: wave w takes heads 32 (w / 4) .. + 31 of the 32-slot tiles w % 4, w % 4 + 4, ...,
// so each wave holds half the dQI accumulators of the four-wave form and two waves fit
// on each SIMD. The two waves of a tile fetch half its ki rows each into a shared,
// double-buffered LDS tile (one LDS barrier per tile step; every wave runs the same
// number of steps). Sweep 1 leaves the two half sums of I per slot in LDS; the row's
// max and sum of exp(I - max) come from block reductions afterwards. Sweep 2 takes
// the dots with slots as M, as in the four-wave key-major form.
template <int IO>
__global__ __launch_bounds__(512) void sli_student_hs_kernel(SliArgs a) {
  constexpr int DI = 128;
  constexpr int QIP = DI + 8;          // ki row pitch: odd count of 16-byte units
  constexpr int KK = DI / 16;          // k-steps of the dots
  constexpr int NCB = DI / 32;         // 32-column blocks of dQI
  constexpr int NW = 8, NP = 4;        // waves, tile streams
  constexpr int LPW = SBT / 2 * (DI / 8) / 64;   // 16-byte ki chunks per lane (half a tile)
  __shared__ __attribute__((aligned(16))) uint16_t KIw[NP][2][SBT * QIP];
  __shared__ __attribute__((aligned(16))) float s_i[SLI_MAX_SLOTS];    // I (heads 0-31 part), then I, dI
  __shared__ __attribute__((aligned(16))) float s_ip[SLI_MAX_SLOTS];   // I (heads 32-63 part)
  __shared__ __attribute__((aligned(16))) uint32_t s_dih[SLI_MAX_SLOTS / 2], s_dil[SLI_MAX_SLOTS / 2];
  __shared__ float s_red[NW];
  __shared__ float s_dw[NP][64];
  static_assert(sizeof(KIw) >= 64 * DI * 4, "the dQI sum fits the ki tiles");

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hh = wave >> 2, pi = wave & 3;   // head half, tile stream
  const int r = blockIdx.x;
  int b, s1;
  const int n = row_slots(a, r, b, s1);
  const int G = a.nidx1;
  uint16_t* dqio = reinterpret_cast<uint16_t*>(a.dqi);
  const int64_t qrow = (int64_t)r * G;
  auto store_w = [&](int g, float v) {
    if (a.wdt == DSA_DTYPE_F32) reinterpret_cast<float*>(a.dw)[qrow + g] = v;
    else if (a.wdt == DSA_DTYPE_BF16) reinterpret_cast<uint16_t*>(a.dw)[qrow + g] = f32_to_bf16_rne(v);
    else reinterpret_cast<uint16_t*>(a.dw)[qrow + g] = f32_to_f16_rne(v);
  };
  const bool lse_only = a.lse_max != nullptr;
  if (lse_only && n == 0) {
    if (tid == 0) { a.lse_max[r] = -INFINITY; a.lse_sum[r] = 0.f; }
    return;
  }
  if (n == 0 || (a.isum && !(a.isum[r] > 0.f))) {
    for (int i = tid; i < G * DI; i += 512) dqio[qrow * DI + i] = 0;
    for (int g = tid; g < G; g += 512) store_w(g, 0.f);
    if (tid == 0) a.row_loss[r] = 0.f;
    return;
  }
  const uint16_t* qib = reinterpret_cast<const uint16_t*>(a.qi);
  const uint16_t* kib = reinterpret_cast<const uint16_t*>(a.ki);
  // this wave's heads: qi fragments (head 32 hh + lane % 32, k = 16 kk + 8 (lane / 32) ..)
  // and the weight of head 32 hh + m32_row(e, lane)
  const int gq = 32 * hh + (lane & 31);
  uint4 qf[KK];
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) qf[kk] = ldg16_or0(gq < G, qib + (qrow + gq) * DI + kk * 16 + (lane >> 5) * 8);
  float wv[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int g = 32 * hh + m32_row(e, lane);
    wv[e] = g < G ? ld_w(a.w, a.wdt, qrow + g) : 0.f;
  }
  const int32_t* ids = a.sidx ? a.sidx + (int64_t)r * a.topk : nullptr;
  const int ntiles = (n + SBT - 1) / SBT;
  const int nsteps = (ntiles + NP - 1) / NP;

  // half hh of tile t: rows 16 hh .. 16 hh + 15; lane l holds chunks l + 64 j
  int idn = 0;   // sparse mode: ids of the next tile to fetch (slot lane % 32), one tile ahead
  auto load_ids = [&](int t) {
    const int sl = t * SBT + (lane & 31);
    if (ids) idn = sl < n ? ids[sl] : 0;
  };
  uint4 stg[LPW];
  auto fetch = [&](int t) {
    const int t0 = t * SBT, nv = n - t0 < SBT ? n - t0 : SBT;
#pragma unroll
    for (int j = 0; j < LPW; ++j) {
      const int i = lane + 64 * j;
      const int row = 16 * hh + i / (DI / 8), c = (i % (DI / 8)) * 8;
      const int key = ids ? clip_id(__shfl(idn, row), a.s2) : t0 + row;
      stg[j] = ldg16_or0(row < nv, kib + ((int64_t)b * a.s2 + key) * DI + c);
    }
  };
  auto commit = [&](uint16_t* kt) {
#pragma unroll
    for (int j = 0; j < LPW; ++j) {
      const int i = lane + 64 * j;
      *reinterpret_cast<uint4*>(&kt[(16 * hh + i / (DI / 8)) * QIP + (i % (DI / 8)) * 8]) = stg[j];
    }
  };
  auto first_fetch = [&]() {
    if (pi < ntiles) {
      load_ids(pi);
      fetch(pi);
      load_ids(pi + NP);
    }
  };
  auto next_fetch = [&](int t) {
    if (t + NP < ntiles) {
      fetch(t + NP);
      load_ids(t + 2 * NP);
    }
  };
  auto bk_read = [&](const uint16_t* kt, uint4 (&bk)[KK]) {
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
      bk[kk] = *reinterpret_cast<const uint4*>(kt + (lane & 31) * QIP + kk * 16 + (lane >> 5) * 8);
  };

  // ---- first sweep: this wave's half of I per slot (heads as M: in-lane sums)
  float* const s_ih = hh == 0 ? s_i : s_ip;
  first_fetch();
  for (int st = 0; st < nsteps; ++st) {
    const int t = pi + NP * st;
    uint16_t* const kt = KIw[pi][st & 1];
    if (t < ntiles) commit(kt);
    lds_barrier();   // both halves of the tile (the buffer's previous tile was read before the last barrier)
    next_fetch(t);
    if (t < ntiles) {
      uint4 bk[KK];
      bk_read(kt, bk);
      f32x16 acc = {};
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) acc = Mfma<IO>::m32(qf[kk], bk[kk], acc);
      float p4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int e = 0; e < 16; ++e) p4[e & 3] += fmaxf(acc[e], 0.f) * wv[e];
      const float iv = add_half_swap((p4[0] + p4[1]) + (p4[2] + p4[3]));
      const int t0 = t * SBT, slot = lane & 31;
      if (lane < 32 && t0 + slot < n) s_ih[t0 + slot] = iv;
    }
  }
  __syncthreads();
  // I = both halves; the row's max and sum of exp(I - max)
  auto block_red = [&](float v, bool is_max) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const float u = __shfl_xor(v, o);
      v = is_max ? fmaxf(v, u) : v + u;
    }
    if (lane == 0) s_red[wave] = v;
    __syncthreads();
    float t = s_red[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) t = is_max ? fmaxf(t, s_red[w]) : t + s_red[w];
    __syncthreads();
    return t;
  };
  float lm = -INFINITY;
  for (int k = tid; k < n; k += 512) {
    const float iv = s_i[k] + s_ip[k];
    s_i[k] = iv;
    lm = fmaxf(lm, iv);
  }
  float mx, inv;
  if (a.isum) {
    mx = a.imax[r];
    inv = 1.f / fmaxf(a.isum[r], SEPS);
  } else {
    mx = block_red(lm, true);   // its barriers also publish every I
    float le = 0.f;
    for (int k = tid; k < n; k += 512) le += expf(s_i[k] - mx);
    const float es = block_red(le, false);
    if (lse_only) {
      if (tid == 0) { a.lse_max[r] = mx; a.lse_sum[r] = es; }
      return;
    }
    inv = ids ? 1.f / (es + SEPS) : 1.f / fmaxf(es, SEPS);
  }
  // dI, the row's KL term, and dI per key for the key-major dKI pass
  float ls = 0.f;
  for (int k = tid; k < n; k += 512) {
    const float sv = expf(s_i[k] - mx) * inv;
    const float pv = a.p[(int64_t)r * a.topk + k];
    const float pc = fmaxf(pv, SEPS), sc = fmaxf(sv, SEPS);
    ls += pc * (logf(pc) - logf(sc));
    s_i[k] = sv - pv;
    if (ids) unsafeAtomicAdd(a.dib + (int64_t)r * a.dib_ld + slot_key(a, ids, k), sv - pv);
    else a.p[(int64_t)r * a.topk + k] = sv - pv;
  }
  const float row_loss = block_red(ls, false);   // its barriers also publish every dI
  if (tid == 0) a.row_loss[r] = row_loss;
  // dI of slot pairs as packed hi / lo parts, and dI = 0 past the row's slots
  for (int m = tid; m < ntiles * (SBT / 2); m += 512) {
    const float d0 = 2 * m < n ? s_i[2 * m] : 0.f, d1 = 2 * m + 1 < n ? s_i[2 * m + 1] : 0.f;
    const uint16_t h0 = from_f32<IO>(d0), h1 = from_f32<IO>(d1);
    const uint16_t l0 = from_f32<IO>(d0 - to_f32<IO>(h0)), l1 = from_f32<IO>(d1 - to_f32<IO>(h1));
    s_dih[m] = h0 | ((uint32_t)h1 << 16);
    s_dil[m] = l0 | ((uint32_t)l1 << 16);
    if (2 * m >= n) s_i[2 * m] = 0.f;
    if (2 * m + 1 >= n) s_i[2 * m + 1] = 0.f;
  }
  __syncthreads();

  // ---- second sweep: dots with slots as M (element e: slot m32_row(e, lane), head
  // 32 hh + lane % 32); dQI[head, :] += (mask dI)[head, slots] ki[slots, :], the
  // operand from the masked dI pairs after one half swap per register pair
  f32x16 dq[NCB];
#pragma unroll
  for (int j = 0; j < NCB; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) dq[j][e] = 0.f;
  float dwh = 0.f;   // dW of head 32 hh + lane % 32 over this lane's slots
  first_fetch();
  for (int st = 0; st < nsteps; ++st) {
    const int t = pi + NP * st;
    uint16_t* const kt = KIw[pi][st & 1];
    if (t < ntiles) commit(kt);
    lds_barrier();
    next_fetch(t);
    if (t < ntiles) {
      uint4 bk[KK];
      bk_read(kt, bk);
      f32x16 acc = {};
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) acc = Mfma<IO>::m32(bk[kk], qf[kk], acc);
      const int sb = t * SBT + 4 * (lane >> 5);   // group g: slots sb + 8 g + 0 .. 3
      float dv[16];
      uint32_t hp[8], lp[8];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 f = *reinterpret_cast<const float4*>(&s_i[sb + 8 * g]);
        dv[4 * g] = f.x; dv[4 * g + 1] = f.y; dv[4 * g + 2] = f.z; dv[4 * g + 3] = f.w;
        const uint2 h = *reinterpret_cast<const uint2*>(&s_dih[(sb + 8 * g) / 2]);
        const uint2 l = *reinterpret_cast<const uint2*>(&s_dil[(sb + 8 * g) / 2]);
        hp[2 * g] = h.x; hp[2 * g + 1] = h.y;
        lp[2 * g] = l.x; lp[2 * g + 1] = l.y;
      }
      float dw = 0.f;
#pragma unroll
      for (int e = 0; e < 16; ++e) dw += fmaxf(acc[e], 0.f) * dv[e];
      dwh += dw;
#pragma unroll
      for (int kq = 0; kq < SBT / 16; ++kq) {
        uint32_t xh[2], yh[2], xl[2], yl[2];
#pragma unroll
        for (int pp = 0; pp < 2; ++pp) {
          const int ex = 8 * kq + 2 * pp, ey = ex + 4;
          const uint32_t mx2 = (acc[ex] > 0.f ? 0xFFFFu : 0u) | (acc[ex + 1] > 0.f ? 0xFFFF0000u : 0u);
          const uint32_t my2 = (acc[ey] > 0.f ? 0xFFFFu : 0u) | (acc[ey + 1] > 0.f ? 0xFFFF0000u : 0u);
          xh[pp] = mx2 & hp[4 * kq + pp];
          xl[pp] = mx2 & lp[4 * kq + pp];
          yh[pp] = my2 & hp[4 * kq + 2 + pp];
          yl[pp] = my2 & lp[4 * kq + 2 + pp];
        }
        swap_halves(xh[0], yh[0]);
        swap_halves(xh[1], yh[1]);
        swap_halves(xl[0], yl[0]);
        swap_halves(xl[1], yl[1]);
        const uint4 ah = make_uint4(xh[0], xh[1], yh[0], yh[1]), al = make_uint4(xl[0], xl[1], yl[0], yl[1]);
#pragma unroll
        for (int j = 0; j < NCB; ++j) {
          const uint4 bv = s_tr_frag(kt, QIP, 32 * j, kq * 16, lane);
          dq[j] = Mfma<IO>::m32(ah, bv, dq[j]);
          dq[j] = Mfma<IO>::m32(al, bv, dq[j]);
        }
      }
    }
  }
  // ---- dW per head over the tile streams; dQI (times the factored w) summed in stream
  // order in LDS (the ki tiles are free)
  {
    const float v = dwh + __shfl_xor(dwh, 32);
    if (lane < 32) s_dw[pi][32 * hh + lane] = v;
  }
  float* const qacc = reinterpret_cast<float*>(&KIw[0][0][0]);   // [64][DI]
  __syncthreads();
#pragma unroll 1
  for (int p = 0; p < NP; ++p) {
    if (pi == p) {
#pragma unroll
      for (int j = 0; j < NCB; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          float* q = qacc + (32 * hh + m32_row(e, lane)) * DI + 32 * j + (lane & 31);
          const float v = dq[j][e] * wv[e];
          *q = (p == 0 ? 0.f : *q) + v;
        }
    }
    __syncthreads();
  }
  for (int i = tid; i < G * DI; i += 512) dqio[qrow * DI + i] = from_f32<IO>(qacc[i]);
  for (int g = tid; g < G; g += 512) store_w(g, (s_dw[0][g] + s_dw[1][g]) + (s_dw[2][g] + s_dw[3][g]));
}

// Key-major dKI: dKI[t, col] = sum over the rows r and heads g of ds[r, g, t] qi[r, g, col],
// ds = dI[r, t] w[r, g] [qi[r, g] . ki[t] > 0], with dI[r, t] the student's dI summed over
// the row's slots that hold key t (zero for keys the row does not use). In dense mode a row's
// keys are t < min(s1 + act_k - act_q + 1, S2) (slot t = key t) and dI sits in p; in sparse
// mode every key of the row is read from the dense buffer dib. One work-group per (tile of
// 128 keys, group of KM_RPG rows, batch); wave w owns keys 32w .. 32w + 31 of the tile
// and keeps their ki fragments in registers. Per row the dots are recomputed with heads
// as M (qi and w staged in LDS, double-buffered: the next row's arrive in registers
// while this row computes); in that accumulator layout a lane holds 16 heads of one
// key, and one v_permlane32_swap per register pair turns two groups of four heads into
// the ds^T operand [key, 8 heads] of the dKI product, which accumulates in registers
// over the group's rows. One fp32 atomic add per element and row group at the end.
constexpr int KM_RPG = 32;   // rows per work-group
template <int IO, int MT, bool EW>
__global__ __launch_bounds__(256) void sli_dki_km_kernel(SliArgs a) {
  constexpr int DI = 128, GP = 32 * MT, QIP = DI + 8, KK = DI / 16, NCB = DI / 32;
  constexpr int QL = GP * (DI / 8) / 256;   // 16-byte qi chunks per thread and row
  __shared__ __attribute__((aligned(16))) uint16_t QIs[2][GP * QIP];
  __shared__ __attribute__((aligned(16))) float Ws[2][GP];
  __shared__ __attribute__((aligned(16))) uint16_t Ws16[EW ? 2 : 1][EW ? GP : 4];   // EW: the weights' own bits
  __shared__ __attribute__((aligned(16))) float s_di[EW ? 4 : 1][32];               // EW: dI of the wave's keys
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b = blockIdx.z;
  const int k0 = blockIdx.x * 128 + 32 * wave;   // this wave's first key
  const int key = k0 + (lane & 31);
  const int G = a.nidx1;
  const int aq = a.act_q[b], ak = a.act_k[b];
  const int off = ak - aq + 1;                    // row s1 sees keys < min(s1 + off, S2)
  // the rows of this group that see any key of the tile
  int s_lo = blockIdx.y * KM_RPG, s_hi = s_lo + KM_RPG;
  s_hi = s_hi < aq ? s_hi : aq;
  s_hi = s_hi < a.s1 ? s_hi : a.s1;
  const bool dense = a.sidx == nullptr;
  const int first_vis = blockIdx.x * 128 - off + 1;   // smallest s1 with s1 + off > tile start
  if (dense) s_lo = s_lo > first_vis ? s_lo : first_vis;
  if (s_lo >= s_hi) return;
  const uint16_t* qib = reinterpret_cast<const uint16_t*>(a.qi);
  const uint16_t* kib = reinterpret_cast<const uint16_t*>(a.ki);
  const uint4 z4 = make_uint4(0, 0, 0, 0);
  // ki fragments of this wave's keys (B of the dots: key lane % 32, k = 16 kk + 8 (lane / 32) ..)
  uint4 bk[KK];
#pragma unroll
  for (int kk = 0; kk < KK; ++kk)
    bk[kk] = ldg16_or0(key < a.s2, kib + ((int64_t)b * a.s2 + key) * DI + kk * 16 + (lane >> 5) * 8);
  uint4 qst[QL];
  float wst = 0.f, dst_ = 0.f;
  uint16_t wst16 = 0;
  bool okst = true;   // rows with an empty indexer softmax have no dI
  auto stage = [&](int s1) {
    okst = !(a.isum && !(a.isum[(int64_t)b * a.s1 + s1] > 0.f));
    const int64_t qrow = ((int64_t)b * a.s1 + s1) * G;
#pragma unroll
    for (int j = 0; j < QL; ++j) {
      const int i = tid + 256 * j;
      const int g = i / (DI / 8), c = (i % (DI / 8)) * 8;
      qst[j] = ldg16_or0(g < G, qib + (qrow + g) * DI + c);
    }
    if (tid < GP) {
      if constexpr (EW) wst16 = tid < G ? reinterpret_cast<const uint16_t*>(a.w)[qrow + tid] : (uint16_t)0;
      else wst = tid < G ? ld_w(a.w, a.wdt, qrow + tid) : 0.f;
    }
    const int n = dense && s1 + off < a.s2 ? s1 + off : a.s2;   // the row's keys
    dst_ = key < n ? a.dib[((int64_t)b * a.s1 + s1) * a.dib_ld + key] : 0.f;
  };
  auto put = [&](int buf) {
#pragma unroll
    for (int j = 0; j < QL; ++j) {
      const int i = tid + 256 * j;
      *reinterpret_cast<uint4*>(&QIs[buf][(i / (DI / 8)) * QIP + (i % (DI / 8)) * 8]) = qst[j];
    }
    if (tid < GP) {
      if constexpr (EW) Ws16[buf][tid] = wst16;
      else Ws[buf][tid] = wst;
    }
  };
  f32x16 c[NCB];
#pragma unroll
  for (int j = 0; j < NCB; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) c[j][e] = 0.f;
  stage(s_lo);
  for (int s1 = s_lo; s1 < s_hi; ++s1) {
    const int buf = (s1 - s_lo) & 1;
    put(buf);
    const float di = dst_;   // dI of this lane's key (0 past the row's keys)
    const bool ok = __builtin_amdgcn_readfirstlane((int)okst) != 0;   // the same for every lane
    if (s1 + 1 < s_hi) stage(s1 + 1);
    lds_barrier();   // this row's qi and w (the other buffer is rewritten only after the next barrier)
    if (!ok) continue;
    const uint16_t* q = QIs[buf];
    // dots[head, key]: element e of mt -> head 32 mt + m32_row(e, lane), key lane % 32
    f32x16 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[mt][e] = 0.f;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const uint4 af = *reinterpret_cast<const uint4*>(q + (32 * mt + (lane & 31)) * QIP + kk * 16 + (lane >> 5) * 8);
        acc[mt] = Mfma<IO>::m32(af, bk[kk], acc[mt]);
      }
    if constexpr (EW) {
      // weights in the io dtype: [dot > 0] w is exact in it, so dKI[key, :] += dI[key]
      // sum_h ([dot > 0] w)[key, h] qi[h, :] takes one MFMA per k-step, and dI scales the
      // product in fp32 (no hi / lo split)
      if (lane < 32) s_di[wave][lane] = di;
      float dv[16];   // dI of key m32_row(e, lane): groups of four consecutive keys
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 f = *reinterpret_cast<const float4*>(&s_di[wave][8 * g + 4 * (lane >> 5)]);
        dv[4 * g] = f.x; dv[4 * g + 1] = f.y; dv[4 * g + 2] = f.z; dv[4 * g + 3] = f.w;
      }
      uint32_t mp[MT][4][2];   // group q of mt: heads 32 mt + 8 q + 4 (lane / 32) + 0 .. 3
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int qg = 0; qg < 4; ++qg) {
          const uint2 wp = *reinterpret_cast<const uint2*>(&Ws16[buf][32 * mt + 8 * qg + 4 * (lane >> 5)]);
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const uint32_t m = (acc[mt][4 * qg + 2 * h] > 0.f ? 0xFFFFu : 0u) |
                               (acc[mt][4 * qg + 2 * h + 1] > 0.f ? 0xFFFF0000u : 0u);
            mp[mt][qg][h] = m & (h == 0 ? wp.x : wp.y);
          }
        }
      uint4 aw[GP / 16];
#pragma unroll
      for (int kq = 0; kq < GP / 16; ++kq) {
        const int mt = kq / 2, g0 = 2 * (kq % 2);
        uint32_t x0 = mp[mt][g0][0], x1 = mp[mt][g0][1], y0 = mp[mt][g0 + 1][0], y1 = mp[mt][g0 + 1][1];
        swap_halves(x0, y0);
        swap_halves(x1, y1);
        aw[kq] = make_uint4(x0, x1, y0, y1);
      }
#pragma unroll
      for (int j = 0; j < NCB; ++j) {
        f32x16 t = {};
#pragma unroll
        for (int kq = 0; kq < GP / 16; ++kq) t = Mfma<IO>::m32(aw[kq], s_tr_frag(q, QIP, 32 * j, kq * 16, lane), t);
#pragma unroll
        for (int e = 0; e < 16; ++e) c[j][e] += dv[e] * t[e];
      }
      continue;
    }
    // ds in the io dtype (hi, and lo = the rounding error), packed four heads per
    // register pair: group q of mt holds heads 32 mt + 8 q + 4 (lane / 32) + 0 .. 3
    uint32_t hp[MT][4][2], lp[MT][4][2];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int qg = 0; qg < 4; ++qg) {
        const float4 w4 = *reinterpret_cast<const float4*>(&Ws[buf][32 * mt + 8 * qg + 4 * (lane >> 5)]);
        const float wq[4] = {w4.x, w4.y, w4.z, w4.w};
        float dsv[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) dsv[u] = acc[mt][4 * qg + u] > 0.f ? di * wq[u] : 0.f;
        uint16_t hi[4], lo[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          hi[u] = from_f32<IO>(dsv[u]);
          lo[u] = from_f32<IO>(dsv[u] - to_f32<IO>(hi[u]));
        }
        hp[mt][qg][0] = hi[0] | ((uint32_t)hi[1] << 16);
        hp[mt][qg][1] = hi[2] | ((uint32_t)hi[3] << 16);
        lp[mt][qg][0] = lo[0] | ((uint32_t)lo[1] << 16);
        lp[mt][qg][1] = lo[2] | ((uint32_t)lo[3] << 16);
      }
    // dKI[key, col] += sum over heads: k-step kq covers heads 16 kq .. 16 kq + 15 (groups
    // 2 (kq % 2) and 2 (kq % 2) + 1 of mt = kq / 2); after the half swap lane l holds
    // heads 16 kq + 8 (l / 32) + 0 .. 7 of key l % 32, the A operand
#pragma unroll
    for (int kq = 0; kq < GP / 16; ++kq) {
      const int mt = kq / 2, g0 = 2 * (kq % 2);
      uint32_t xh0 = hp[mt][g0][0], xh1 = hp[mt][g0][1], yh0 = hp[mt][g0 + 1][0], yh1 = hp[mt][g0 + 1][1];
      uint32_t xl0 = lp[mt][g0][0], xl1 = lp[mt][g0][1], yl0 = lp[mt][g0 + 1][0], yl1 = lp[mt][g0 + 1][1];
      swap_halves(xh0, yh0);
      swap_halves(xh1, yh1);
      swap_halves(xl0, yl0);
      swap_halves(xl1, yl1);
      const uint4 ah = make_uint4(xh0, xh1, yh0, yh1), al = make_uint4(xl0, xl1, yl0, yl1);
#pragma unroll
      for (int j = 0; j < NCB; ++j) {
        const uint4 bv = s_tr_frag(q, QIP, 32 * j, kq * 16, lane);
        c[j] = Mfma<IO>::m32(ah, bv, c[j]);
        c[j] = Mfma<IO>::m32(al, bv, c[j]);
      }
    }
  }
  // element e of c[j]: key k0 + m32_row(e, lane), column 32 j + lane % 32
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int kt = k0 + m32_row(e, lane);
    if (kt < a.s2) {
      float* dst = a.dki_acc + ((int64_t)b * a.s2 + kt) * DI + (lane & 31);
#pragma unroll
      for (int j = 0; j < NCB; ++j) unsafeAtomicAdd(dst + 32 * j, c[j][e]);
    }
  }
}

// dKI accumulator -> io dtype; the loss as the row-ordered sum of the row losses
template <int IO>
__global__ void sli_finish_kernel(SliArgs a, int64_t n4, int rows) {
  const float4* src = reinterpret_cast<const float4*>(a.dki_acc);
  uint2* dst = reinterpret_cast<uint2*>(a.dki);
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (int64_t)gridDim.x * blockDim.x) {
    const float4 v = src[i];
    dst[i] = make_uint2(pack2<IO>(v.x, v.y), pack2<IO>(v.z, v.w));
  }
  if (blockIdx.x == 0) {
    __shared__ float part[256];
    float s = 0.f;
    const int per = (rows + 255) / 256;
    for (int i = threadIdx.x * per; i < (threadIdx.x + 1) * per && i < rows; ++i) s += a.row_loss[i];
    part[threadIdx.x] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
      float t = 0.f;
      for (int i = 0; i < 256; ++i) t += part[i];
      a.loss[0] = t;
    }
  }
}

// head blocks per pass: the smallest of 1, 2, 4 covering Nidx1 / 32 whose qi block
// 32 NGB x DI stays within SLI_MAX_GD elements of LDS; otherwise passes of 64 heads.
// Rows of more than SLI_MAX_SLOTS slots keep I / dI in the workspace (BIG).
template <int IO, int DI, bool BIG>
void launch_student_big(const SliArgs& a, int rows, hipStream_t s) {
  const int ngb = (a.nidx1 + 31) / 32;
  if (ngb <= 1)
    hipLaunchKernelGGL((sli_student_kernel<IO, DI, 1, 1, BIG>), dim3(rows), dim3(256), 0, s, a);
  else if (ngb <= 2)
    hipLaunchKernelGGL((sli_student_kernel<IO, DI, 2, 1, BIG>), dim3(rows), dim3(256), 0, s, a);
  else if constexpr (128 * DI <= SLI_MAX_GD)
    hipLaunchKernelGGL((sli_student_kernel<IO, DI, 4, 1, BIG>), dim3(rows), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((sli_student_kernel<IO, DI, 2, 2, BIG>), dim3(rows), dim3(256), 0, s, a);
}

// the key-major dKI pass; the exact-weight form when the weights are in the io dtype
template <int IO, int MT>
void launch_km(const SliArgs& a, hipStream_t s) {
  const dim3 g((a.s2 + 127) / 128, (a.s1 + KM_RPG - 1) / KM_RPG, a.batch);
  const bool ew = a.wdt == (IO == IO_BF16 ? DSA_DTYPE_BF16 : DSA_DTYPE_F16);
  if (ew) hipLaunchKernelGGL((sli_dki_km_kernel<IO, MT, true>), g, dim3(256), 0, s, a);
  else hipLaunchKernelGGL((sli_dki_km_kernel<IO, MT, false>), g, dim3(256), 0, s, a);
}

template <int IO, int DI>
void launch_student(const SliArgs& a, int rows, hipStream_t s) {
  if constexpr (DI == 128) {
    // D_idx = 128, Nidx1 <= 64, rows within SLI_MAX_SLOTS slots: the wave-per-tile form
    if (a.nidx1 <= 64 && a.topk <= SLI_MAX_SLOTS) {
      if (a.nidx1 > 32 && (a.dki_km || a.lse_max)) {
        // 33 - 64 heads: the eight-wave head-split form (stats only, or dKI left to the key-major pass)
        hipLaunchKernelGGL((sli_student_hs_kernel<IO>), dim3(rows), dim3(512), 0, s, a);
        if (a.dki_km) launch_km<IO, 2>(a, s);
        return;
      }
      if (a.dki_km) {   // <= 32 heads here (more take the head-split form above)
        hipLaunchKernelGGL((sli_student_wt_kernel<IO, 1, true>), dim3(rows), dim3(256), 0, s, a);
        launch_km<IO, 1>(a, s);
      } else {
        if (a.nidx1 <= 32) hipLaunchKernelGGL((sli_student_wt_kernel<IO, 1, false>), dim3(rows), dim3(256), 0, s, a);
        else hipLaunchKernelGGL((sli_student_wt_kernel<IO, 2, false>), dim3(rows), dim3(256), 0, s, a);
      }
      return;
    }
  }
  if (a.topk > SLI_MAX_SLOTS && !a.lse_max) launch_student_big<IO, DI, true>(a, rows, s);
  else launch_student_big<IO, DI, false>(a, rows, s);
}

template <int IO>
hipError_t launch_sli_io(const SliArgs& a, hipStream_t s) {
  const int rows = a.batch * a.s1;
  if (a.lse_max) {   // stats only: the student's first pass
    switch (a.didx) {
      case 128: launch_student<IO, 128>(a, rows, s); break;
      case 256: launch_student<IO, 256>(a, rows, s); break;
      case 512: launch_student<IO, 512>(a, rows, s); break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  const dim3 tgrid(rows, (a.n1 + SBH - 1) / SBH);
  if (a.n2 > 1) {
    // one-dimensional grids rounded up to whole XCD rounds (the kernel maps the ids)
    const int nrb = (a.s1 + 31) / 32;
    const int64_t n4 = (int64_t)a.batch * nrb * ((a.s2 + 127) / 128), n2 = (int64_t)a.batch * nrb * ((a.s2 + 63) / 64);
    const dim3 g4((unsigned)((n4 + 7) / 8 * 8)), g2((unsigned)((n2 + 7) / 8 * 8));
    switch (a.d + a.dr) {
      case 128: hipLaunchKernelGGL((sli_teacher_heads_kernel<IO, 128, 4>), g4, dim3(256), 0, s, a); break;
      case 192: hipLaunchKernelGGL((sli_teacher_heads_kernel<IO, 192, 4>), g4, dim3(256), 0, s, a); break;
      case 256: hipLaunchKernelGGL((sli_teacher_heads_kernel<IO, 256, 4>), g4, dim3(256), 0, s, a); break;
      case 320: hipLaunchKernelGGL((sli_teacher_heads_kernel<IO, 320, 4>), g4, dim3(256), 0, s, a); break;
      case 512: hipLaunchKernelGGL((sli_teacher_heads_kernel<IO, 512, 2>), g2, dim3(128), 0, s, a); break;
      case 576: hipLaunchKernelGGL((sli_teacher_heads_kernel<IO, 576, 2>), g2, dim3(128), 0, s, a); break;
      default: return hipErrorInvalidValue;
    }
  } else if (a.dr == DR_TEACH && (a.d == 128 || a.d == 256 || a.d == 512)) {
    // one key head with rope: the attention kernel's S path (direct-to-LDS gather ring,
    // all heads of a row per work-group) writes p
    SfaArgs t{a.q, a.qr, a.k, a.kr, a.io, a.sidx, a.topk, 1, nullptr, 0, 0, nullptr, nullptr, a.act_q, a.act_k,
              a.batch, rows, a.n1, a.d, a.dr, a.s2, (int64_t)a.batch * a.s2, 3, a.scale, nullptr, nullptr, nullptr,
              a.tok_ws, sfa_token_ws_bytes(rows, a.topk, 1), 1};
    t.t_p = a.p;
    t.t_ld = a.topk;
    t.t_max = a.sm_max;
    t.t_sum = a.sm_sum;
    t.t_s1 = a.s1;
    const hipError_t e = launch_sfa_teacher(t, s);
    if (e != hipSuccess) return e;
  } else switch (a.d + a.dr) {
    case 128: hipLaunchKernelGGL((sli_teacher_kernel<IO, 128>), tgrid, dim3(256), 0, s, a); break;
    case 192: hipLaunchKernelGGL((sli_teacher_kernel<IO, 192>), tgrid, dim3(256), 0, s, a); break;
    case 256: hipLaunchKernelGGL((sli_teacher_kernel<IO, 256>), tgrid, dim3(256), 0, s, a); break;
    case 320: hipLaunchKernelGGL((sli_teacher_kernel<IO, 320>), tgrid, dim3(256), 0, s, a); break;
    case 512: hipLaunchKernelGGL((sli_teacher_kernel<IO, 512>), tgrid, dim3(256), 0, s, a); break;
    case 576: hipLaunchKernelGGL((sli_teacher_kernel<IO, 576>), tgrid, dim3(256), 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  switch (a.didx) {
    case 128: launch_student<IO, 128>(a, rows, s); break;
    case 256: launch_student<IO, 256>(a, rows, s); break;
    case 512: launch_student<IO, 512>(a, rows, s); break;
    default: return hipErrorInvalidValue;
  }
  const int64_t n4 = (int64_t)a.batch * a.s2 * a.didx / 4;
  const int blocks = (int)((n4 + 255) / 256 < 4096 ? ((n4 + 255) / 256 > 0 ? (n4 + 255) / 256 : 1) : 4096);
  hipLaunchKernelGGL((sli_finish_kernel<IO>), dim3(blocks), dim3(256), 0, s, a, n4, rows);
  return hipGetLastError();
}

}  // namespace
}  // namespace dsa

int sli_km_sparse_ld(int rows, int topk, int s2, int didx) {
  // the key-major pass reads every key of a row: worth it while the rows use a large
  // share of the keys (it replaces D_idx fp32 atomics per slot)
  if (didx != 128 || topk > dsa::SLI_MAX_SLOTS || (int64_t)s2 > 4LL * topk) return 0;
  if ((int64_t)rows * s2 * 4 > ((int64_t)512 << 20)) return 0;
  return s2;
}

size_t sli_grad_workspace_bytes(int rows, int topk, int64_t key_rows, int didx, int km_ld) {
  return dsa::salign((size_t)rows * topk * 4) + dsa::salign((size_t)key_rows * didx * 4) +
         dsa::salign((size_t)rows * km_ld * 4) +
         dsa::salign((size_t)rows * 4) + (topk > dsa::SLI_MAX_SLOTS ? dsa::salign((size_t)rows * topk * 4) : 0) +
         dsa::salign(sfa_token_ws_bytes(rows > 0 ? rows : 1, topk, 1));
}

bool sli_grad_supported(int d, int dr, int nidx1, int didx, int topk) {
  const int dt = d + dr;
  const bool dt_ok = dt == 128 || dt == 192 || dt == 256 || dt == 320 || dt == 512 || dt == 576;
  const bool di_ok = didx == 128 || didx == 256 || didx == 512;
  return dt_ok && di_ok && nidx1 >= 1 && nidx1 <= 128 && topk >= 1 && topk <= dsa::SLI_MAX_TOPK;
}

namespace {
// workspace: teacher sums [rows, topk] | dKI accumulator [batch s2, didx] | (sparse
// key-major pass) dI per key [rows, km_ld] | row losses | (rows of more than SLI_MAX_SLOTS
// slots) I / dI [rows, topk] | the teacher's token lists
hipError_t run_sli(dsa::SliArgs a, void* ws, int km_ld, hipStream_t s) {
  const int rows = a.batch * a.s1;
  char* base = reinterpret_cast<char*>(ws);
  a.p = reinterpret_cast<float*>(base);
  size_t off = dsa::salign((size_t)rows * a.topk * 4);
  a.dki_acc = reinterpret_cast<float*>(base + off);
  off += dsa::salign((size_t)a.batch * a.s2 * a.didx * 4);
  if (a.sidx) {
    a.dib = reinterpret_cast<float*>(base + off);
    a.dib_ld = km_ld;
    off += dsa::salign((size_t)rows * km_ld * 4);
    a.dki_km = km_ld > 0 && a.didx == 128 && a.nidx1 <= 64 && a.topk <= dsa::SLI_MAX_SLOTS;
  } else {
    a.dib = a.p;
    a.dib_ld = a.topk;
  }
  a.row_loss = reinterpret_cast<float*>(base + off);
  // teacher sums, the dKI accumulator and the dI buffer are contiguous up to the padding
  const int64_t n4 = (int64_t)off / 16;
  size_t off2 = off + dsa::salign((size_t)rows * 4);
  a.ibuf = a.topk > dsa::SLI_MAX_SLOTS ? reinterpret_cast<float*>(base + off2) : nullptr;
  if (a.ibuf) off2 += dsa::salign((size_t)rows * a.topk * 4);
  a.tok_ws = base + off2;
  const int blocks = (int)((n4 + 255) / 256 < 4096 ? ((n4 + 255) / 256 > 0 ? (n4 + 255) / 256 : 1) : 4096);
  hipLaunchKernelGGL(dsa::sli_zero_kernel, dim3(blocks), dim3(256), 0, s, reinterpret_cast<float4*>(base), n4);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return a.io == dsa::IO_BF16 ? dsa::launch_sli_io<dsa::IO_BF16>(a, s) : dsa::launch_sli_io<dsa::IO_F16>(a, s);
}
}  // namespace

bool dense_li_grad_supported(int n1, int n2, int d, int dr, int nidx1, int didx, int s2) {
  if (n2 < 1 || n1 % n2 != 0 || s2 < 1) return false;
  return sli_grad_supported(d, dr, nidx1, didx, 1);
}

hipError_t launch_dense_li_lse(const void* qi, const void* ki, const void* w, int io, int wdt,
                               const int32_t* act_q, const int32_t* act_k, int batch, int s1, int s2,
                               int nidx1, int didx, float* out_max, float* out_sum, hipStream_t s) {
  dsa::SliArgs a{};
  a.qi = qi; a.ki = ki; a.w = w; a.io = io; a.wdt = wdt; a.topk = s2;
  a.act_q = act_q; a.act_k = act_k; a.batch = batch; a.s1 = s1; a.s2 = s2; a.n1 = 1; a.n2 = 1;
  a.nidx1 = nidx1; a.didx = didx; a.lse_max = out_max; a.lse_sum = out_sum;
  return io == dsa::IO_BF16 ? dsa::launch_sli_io<dsa::IO_BF16>(a, s) : dsa::launch_sli_io<dsa::IO_F16>(a, s);
}

hipError_t launch_dense_li_grad(const void* q, const void* k, const void* qr, const void* kr, const void* qi,
                                const void* ki, const void* w, int io, int wdt, const float* sm_max,
                                const float* sm_sum, const float* max_index, const float* sum_index,
                                const int32_t* act_q, const int32_t* act_k, int batch, int s1, int s2, int n1,
                                int n2, int d, int dr, int nidx1, int didx, float scale, void* dqi, void* dki,
                                void* dw, float* loss, void* ws, hipStream_t s) {
  dsa::SliArgs a{q, k, qr, kr, qi, ki, w, io, wdt, nullptr, s2, sm_max, sm_sum, act_q, act_k,
                 batch, s1, s2, n1, d, dr, nidx1, didx, scale, dqi, dki, dw, loss,
                 nullptr, nullptr, nullptr, nullptr, nullptr, n2, max_index, sum_index, nullptr, nullptr};
  a.dki_km = didx == 128 && nidx1 <= 64 && s2 <= dsa::SLI_MAX_SLOTS;
  return run_sli(a, ws, 0, s);
}

hipError_t launch_sli_grad(const void* q, const void* k, const void* qr, const void* kr, const void* qi,
                           const void* ki, const void* w, int io, int wdt, const int32_t* sidx, int topk,
                           const float* sm_max, const float* sm_sum, const int32_t* act_q,
                           const int32_t* act_k, int batch, int s1, int s2, int n1, int d, int dr,
                           int nidx1, int didx, float scale, void* dqi, void* dki, void* dw, float* loss,
                           void* ws, hipStream_t s) {
  dsa::SliArgs a{q, k, qr, kr, qi, ki, w, io, wdt, sidx, topk, sm_max, sm_sum, act_q, act_k,
                 batch, s1, s2, n1, d, dr, nidx1, didx, scale, dqi, dki, dw, loss,
                 nullptr, nullptr, nullptr, nullptr, nullptr};
  a.n2 = 1;
  return run_sli(a, ws, sli_km_sparse_ld(batch * s1, topk, s2, didx), s);
}
