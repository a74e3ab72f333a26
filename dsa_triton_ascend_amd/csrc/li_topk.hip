// Stable top-k over quantised indexer scores, gfx950.
//
// Ordering contract (lightning_indexer_numpy.py:92-105): within the visible
// prefix of a score row, entries are ordered by their 16-bit quantised score
// descending, ties by ascending index; the first min(L, k) are emitted (index
// and quantised score), the other slots get -1 / 0. The reference's device
// path calls mint.topk / mint.sort here (lightning_indexer_triton.py:343-361).
//
// Because every entry is a 16-bit float, (score, index) packs into one unique
// 32-bit key  key = ord16(score) << 16 | (0xFFFF - index)  whose descending
// order is exactly the golden's order (S2 <= 65536). Per score row, one
// work-group of 256 threads:
//   1. L <= k: every visible entry is selected.
//   2. L >  k: radix-select the k-th largest 16-bit score T with two 8-bit
//      LDS histogram passes (the row is re-read from L2), giving cnt_gt
//      (entries > T) and need = k - cnt_gt. Entries > T are appended with an
//      LDS atomic; entries == T are ranked in index order with wave ballots
//      + popcount prefixes and a running block total, the first `need` kept.
//   3. bitonic sort of the k selected unique keys in LDS (descending), then
//      one coalesced pass writes indices and values.
#include "dsa_common.hpp"

namespace dsa {
namespace {

constexpr int TPB = 256;

__device__ __forceinline__ int visible_len(int s1, int aq, int ak, int S2, int mode) {
  int L;
  if (mode == 3) {
    L = ak - aq + s1 + 1;
    L = L < 0 ? 0 : L;
    L = L < S2 ? L : S2;
    L = L < ak ? L : ak;
  } else {
    L = ak < S2 ? ak : S2;
  }
  return L < 0 ? 0 : L;
}

// Block-wide inclusive scan of one uint32 per thread (TPB threads).
__device__ __forceinline__ uint32_t block_incl_scan(uint32_t v, uint32_t* wsum) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    uint32_t n = __shfl_up(v, o);
    if (lane >= o) v += n;
  }
  if (lane == 63) wsum[wave] = v;
  __syncthreads();
  uint32_t off = 0;
#pragma unroll
  for (int w = 0; w < TPB / 64; ++w) off += (w < wave) ? wsum[w] : 0u;
  __syncthreads();
  return v + off;
}

// Given a 256-bin histogram, find the bin holding the k-th largest element:
// returns via LDS the bin and the number of elements in strictly higher bins.
__device__ __forceinline__ void select_bin(const uint32_t* hist, uint32_t k, uint32_t* wsum,
                                           uint32_t* res_bin, uint32_t* res_gt) {
  const int t = threadIdx.x;
  const uint32_t v = hist[255 - t];
  const uint32_t incl = block_incl_scan(v, wsum);
  const uint32_t excl = incl - v;
  if (excl < k && incl >= k) {
    *res_bin = 255 - t;
    *res_gt = excl;
  }
  __syncthreads();
}

__global__ __launch_bounds__(TPB) void li_topk_kernel(LiTopkArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint32_t sel[];  // next_pow2(k) keys
  __shared__ uint32_t hist[256];
  __shared__ uint32_t wsum[TPB / 64];
  __shared__ uint32_t s_bin, s_gt, s_cnt, s_tie;

  const int sr = blockIdx.x;
  const int r = sr / a.n2;
  const int b = batch_of_row(a.row_start, a.batch, r);
  const int s1 = r - a.row_start[b];
  const int aq = a.act_q[b], ak = a.act_k[b];
  const int L = s1 < aq ? visible_len(s1, aq, ak, a.s2, a.sparse_mode) : 0;
  const int k = a.k;
  const int nout = L < k ? L : k;
  int32_t* iout = a.idx + (int64_t)sr * k;
  uint16_t* vout = a.val ? a.val + (int64_t)sr * k : nullptr;
  const uint16_t* row = a.scores + (int64_t)sr * a.ld;
  const int tid = threadIdx.x;

  if (nout == 0) {
    for (int i = tid; i < k; i += TPB) {
      iout[i] = -1;
      if (vout) vout[i] = 0;
    }
    return;
  }

  int P = 1;
  while (P < nout) P <<= 1;

  if (L <= k) {
    for (int i = tid; i < L; i += TPB) sel[i] = (ord16(row[i]) << 16) | (0xFFFFu - (uint32_t)i);
  } else {
    // ---- pass A: high byte of the 16-bit key
    hist[tid] = 0;
    __syncthreads();
    for (int i = tid; i < L; i += TPB) atomicAdd(&hist[ord16(row[i]) >> 8], 1u);
    __syncthreads();
    select_bin(hist, (uint32_t)k, wsum, &s_bin, &s_gt);
    const uint32_t bhi = s_bin, gt_hi = s_gt;
    __syncthreads();
    // ---- pass B: low byte inside the selected high bin
    hist[tid] = 0;
    __syncthreads();
    for (int i = tid; i < L; i += TPB) {
      const uint32_t u = ord16(row[i]);
      if ((u >> 8) == bhi) atomicAdd(&hist[u & 0xFFu], 1u);
    }
    __syncthreads();
    select_bin(hist, (uint32_t)k - gt_hi, wsum, &s_bin, &s_gt);
    const uint32_t T = (bhi << 8) | s_bin;
    const uint32_t cnt_gt = gt_hi + s_gt;
    const uint32_t need = (uint32_t)k - cnt_gt;
    if (tid == 0) { s_cnt = 0; s_tie = 0; }
    __syncthreads();
    // ---- pass C: compaction; ties ranked in index order
    const int lane = tid & 63, wave = tid >> 6;
    for (int base = 0; base < L; base += TPB) {
      const int i = base + tid;
      const uint32_t u = i < L ? ord16(row[i]) : 0u;
      const uint32_t key = (u << 16) | (0xFFFFu - (uint32_t)i);
      if (i < L && u > T) sel[atomicAdd(&s_cnt, 1u)] = key;
      const bool tie = i < L && u == T;
      const uint64_t m = __ballot(tie);
      const uint32_t pre = __popcll(m & ((1ull << lane) - 1ull));
      if (lane == 0) wsum[wave] = (uint32_t)__popcll(m);
      __syncthreads();
      uint32_t woff = 0, tot = 0;
#pragma unroll
      for (int w = 0; w < TPB / 64; ++w) {
        woff += (w < wave) ? wsum[w] : 0u;
        tot += wsum[w];
      }
      const uint32_t rank = s_tie + woff + pre;
      if (tie && rank < need) sel[cnt_gt + rank] = key;
      __syncthreads();
      if (tid == 0) s_tie += tot;
      __syncthreads();
    }
  }
  for (int i = nout + tid; i < P; i += TPB) sel[i] = 0u;  // pads sort last
  __syncthreads();

  // ---- bitonic sort, descending
  for (int k2 = 2; k2 <= P; k2 <<= 1) {
    for (int j = k2 >> 1; j > 0; j >>= 1) {
      for (int i = tid; i < (P >> 1); i += TPB) {
        const int lo = ((i & ~(j - 1)) << 1) | (i & (j - 1));
        const int hi = lo + j;
        const uint32_t x = sel[lo], y = sel[hi];
        const bool desc = (lo & k2) == 0;
        if (desc ? (x < y) : (x > y)) {
          sel[lo] = y;
          sel[hi] = x;
        }
      }
      __syncthreads();
    }
  }

  for (int i = tid; i < k; i += TPB) {
    if (i < nout) {
      const uint32_t key = sel[i];
      iout[i] = (int32_t)(0xFFFFu - (key & 0xFFFFu));
      if (vout) vout[i] = unord16(key >> 16);
    } else {
      iout[i] = -1;
      if (vout) vout[i] = 0;
    }
  }
}

}  // namespace
}  // namespace dsa

size_t li_topk_lds_bytes(int k) {
  size_t P = 1;
  while (P < (size_t)k) P <<= 1;
  return P * 4;
}

hipError_t launch_li_topk(const LiTopkArgs& a, hipStream_t s) {
  const int64_t rows = (int64_t)a.total_rows * a.n2;
  if (rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(dsa::li_topk_kernel, dim3((unsigned)rows), dim3(dsa::TPB),
                     li_topk_lds_bytes(a.k), s, a);
  return hipGetLastError();
}
