// Stable top-k over quantised indexer scores, gfx950.
//
// Ordering contract (lightning_indexer_numpy.py:92-105): within the visible
// prefix of a score row, entries are ordered by their 16-bit quantised score
// descending, ties by ascending index; the first min(L, k) are emitted (index
// and quantised score), the other slots get -1 / 0. The reference's device
// path calls mint.topk / mint.sort here (lightning_indexer_triton.py:343-361).
//
// One 256-thread work-group per score row (any length: indices are 32-bit):
//   1. Thread t owns the contiguous index range [32t, 32t+32) of the row; the
//      16-bit scores are mapped to order-preserving keys u (ord16) and kept in
//      VGPRs (rows longer than 8192 entries are streamed from memory instead, in
//      chunks of 8192).
//   2. L > k: the k-th largest key T is found with two 256-bin LDS histograms:
//      one over the high byte of the keys picks the bin holding the k-th largest
//      (a scan from the top bin), one over the low byte of the keys in that bin
//      picks T; the same scans give the number of keys above T.
//   3. Order-preserving compaction: entries with u > T and the first
//      k - count(u > T) entries with u == T (in index order) are written, in
//      index order, to positions p < k as keys (u << 16 | x); p comes from block
//      exclusive scans of the per-thread counts. Rows of up to 65536 entries carry
//      x = 0xFFFF - index; longer rows (WIDE) carry x = p and keep the 32-bit index
//      in a second LDS array at p (p, like the index, increases along the row).
//   4. A stable LSD radix sort on the 16-bit score (4 passes of 4 bits, digits
//      of the inverted key so larger scores come first; per-thread counter
//      columns in LDS, no atomics). Stability preserves the index order of
//      equal scores, which is exactly the golden's tie rule.
//   5. One pass writes the indices and 16-bit values in rank order.
#include "dsa_common.hpp"

namespace dsa {
namespace {

constexpr int TPB = 256;
constexpr int RPT = 32;                 // row entries per thread held in VGPRs
constexpr int ROW_CACHED = TPB * RPT;   // 8192
// Histogram bins are split into HSUB counters picked by lane % HSUB: scores cluster
// in few high-byte bins, and same-address LDS atomics of one instruction serialise.
constexpr int HSUB = 8;

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

__device__ __forceinline__ uint32_t wave_sum(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Block-wide sum (all threads get the total). `red` holds TPB/64 words.
__device__ __forceinline__ uint32_t block_sum(uint32_t v, uint32_t* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  uint32_t t = 0;
#pragma unroll
  for (int w = 0; w < TPB / 64; ++w) t += red[w];
  return t;
}

// Block-wide exclusive scan; also returns the total.
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t* red, uint32_t* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint32_t x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t n = __shfl_up(x, o);
    if (lane >= o) x += n;
  }
  __syncthreads();
  if (lane == 63) red[wave] = x;
  __syncthreads();
  uint32_t off = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < TPB / 64; ++w) {
    off += (w < wave) ? red[w] : 0u;
    tot += red[w];
  }
  *total = tot;
  return off + x - v;
}

__device__ __forceinline__ void load_keys(const uint16_t* row, int L, int base, uint32_t (&u)[RPT]) {
  const int i0 = base + threadIdx.x * RPT;
  if (i0 + RPT <= L) {
#pragma unroll
    for (int c = 0; c < RPT / 8; ++c) {
      const uint4 v = ldg16(row + i0 + c * 8);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        u[c * 8 + 2 * j] = ord16((uint16_t)(w[j] & 0xFFFFu));
        u[c * 8 + 2 * j + 1] = ord16((uint16_t)(w[j] >> 16));
      }
    }
  } else {
#pragma unroll
    for (int e = 0; e < RPT; ++e) u[e] = (i0 + e < L) ? ord16(row[i0 + e]) : 0u;  // 0 < every real key
  }
}

// Stable LSD radix sort of E keys per thread (blocked: thread t holds ranks
// [E t, E t + E)), ascending on the inverted upper 16 bits = score descending.
template <int E>
__device__ __forceinline__ void radix_sort_desc16(uint32_t (&key)[E], uint32_t* sbuf, uint16_t* cnt,
                                                  uint32_t* red) {
  const int t = threadIdx.x;
#pragma unroll 1
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 16 + 4 * pass;
#pragma unroll
    for (int d = 0; d < 16; ++d) cnt[d * TPB + t] = 0;
    uint16_t lrank[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int d = ((~key[e]) >> shift) & 15;
      const uint16_t r = cnt[d * TPB + t];
      lrank[e] = r;
      cnt[d * TPB + t] = r + 1;
    }
    __syncthreads();
    // exclusive scan over cnt in [digit][thread] order: thread t scans entries 16t..16t+15
    uint32_t loc[16];
    uint32_t s = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      loc[j] = s;
      s += cnt[t * 16 + j];
    }
    uint32_t tot;
    const uint32_t off = block_excl_scan(s, red, &tot);
#pragma unroll
    for (int j = 0; j < 16; ++j) cnt[t * 16 + j] = (uint16_t)(off + loc[j]);
    __syncthreads();
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int d = ((~key[e]) >> shift) & 15;
      sbuf[cnt[d * TPB + t] + lrank[e]] = key[e];
    }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < E; ++e) key[e] = sbuf[E * t + e];
    __syncthreads();
  }
}

template <int E, bool WIDE>
__global__ __launch_bounds__(TPB) void li_topk_kernel(LiTopkArgs a) {
  static_assert(E * TPB <= 65536, "compacted positions are 16-bit");
  __shared__ __attribute__((aligned(16))) uint32_t sbuf[E * TPB];
  __shared__ int32_t sidx[WIDE ? E * TPB : 1];   // WIDE: row index of compacted position p
  __shared__ uint16_t cnt[16 * TPB];
  __shared__ uint32_t red[TPB / 64];
  __shared__ uint32_t hist[256 * HSUB];
  __shared__ uint32_t pick[2];

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
  const int t = threadIdx.x;

  if (nout == 0) {
    for (int i = t; i < k; i += TPB) {
      iout[i] = -1;
      if (vout) vout[i] = 0;
    }
    return;
  }

  // ---- selection + order-preserving compaction into sbuf[0, nout)
  const int nchunks = (L + ROW_CACHED - 1) / ROW_CACHED;
  uint32_t u[RPT];
  if (nchunks == 1) load_keys(row, L, 0, u);
  uint32_t T = 0;  // keys > T are all taken; keys == T up to `need`
  uint32_t need = 0xFFFFFFFFu;
  if (L > k) {
    // 256-bin histogram over (u >> shift) of the keys whose high byte is `match`
    // (every key for the first pass), then a scan from the top bin: the bin that
    // holds the `want`-th largest and the count of keys in higher bins
    auto select_byte = [&](int shift, int match, uint32_t want, uint32_t& above) -> int {
#pragma unroll
      for (int i = 0; i < HSUB; ++i) hist[i * TPB + t] = 0;
      __syncthreads();
      const int sub = t & (HSUB - 1);
#pragma unroll 1
      for (int ch = 0; ch < nchunks; ++ch) {
        if (nchunks > 1) load_keys(row, L, ch * ROW_CACHED, u);
#pragma unroll
        for (int e = 0; e < RPT; ++e)
          if (u[e] != 0u && (match < 0 || (int)(u[e] >> 8) == match))
            atomicAdd(&hist[((u[e] >> shift) & 255u) * HSUB + sub], 1u);
      }
      __syncthreads();
      uint32_t h = 0;   // thread t: bin 255 - t, so the scan runs from the top
#pragma unroll
      for (int i = 0; i < HSUB; ++i) h += hist[(255 - t) * HSUB + i];
      uint32_t tot;
      const uint32_t before = block_excl_scan(h, red, &tot);
      if (before < want && before + h >= want) {
        pick[0] = 255 - t;
        pick[1] = before;
      }
      __syncthreads();
      above = pick[1];
      return (int)pick[0];
    };
    uint32_t above_hi, above_lo;
    const int hb = select_byte(8, -1, (uint32_t)k, above_hi);
    const int lb = select_byte(0, hb, (uint32_t)k - above_hi, above_lo);
    T = ((uint32_t)hb << 8) | (uint32_t)lb;
    need = (uint32_t)k - (above_hi + above_lo);   // keys == T to take, in index order
  }
  // positions: selected-before = greater-before + min(ties-before, need)
  uint32_t run_g = 0, run_e = 0;  // totals of previous chunks
#pragma unroll 1
  for (int ch = 0; ch < nchunks; ++ch) {
    if (nchunks > 1) load_keys(row, L, ch * ROW_CACHED, u);
    uint32_t cg = 0, ce = 0;
#pragma unroll
    for (int e = 0; e < RPT; ++e) {
      cg += u[e] > T ? 1u : 0u;
      ce += (u[e] == T && T != 0) ? 1u : 0u;
    }
    uint32_t tot_g, tot_e;
    uint32_t pg = block_excl_scan(cg, red, &tot_g) + run_g;
    uint32_t pe = block_excl_scan(ce, red, &tot_e) + run_e;
    const int i0 = ch * ROW_CACHED + t * RPT;
#pragma unroll
    for (int e = 0; e < RPT; ++e) {
      // x: the index (rows up to 65536) or the position, whose index goes to sidx
      auto put = [&](uint32_t p) {
        if constexpr (WIDE) {
          sbuf[p] = (u[e] << 16) | p;
          sidx[p] = i0 + e;
        } else {
          sbuf[p] = (u[e] << 16) | (0xFFFFu - (uint32_t)(i0 + e));
        }
      };
      if (u[e] > T) {
        put(pg + (pe < need ? pe : need));
        ++pg;
      } else if (u[e] == T && T != 0) {
        if (pe < need) put(pg + pe);
        ++pe;
      }
    }
    run_g += tot_g;
    run_e += tot_e;
  }
  for (int i = nout + t; i < E * TPB; i += TPB) sbuf[i] = 0u;  // pads sort last
  __syncthreads();

  // ---- stable radix sort of the selected keys, then write in rank order
  uint32_t key[E];
#pragma unroll
  for (int e = 0; e < E; ++e) key[e] = sbuf[E * t + e];
  __syncthreads();
  radix_sort_desc16<E>(key, sbuf, cnt, red);
  // ranks E t .. E t + E - 1 of thread t: their index (or -1) and 16-bit value (or 0)
  int32_t oi[E];
  uint16_t ov[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const bool ok = E * t + e < nout;
    if constexpr (WIDE) oi[e] = ok ? sidx[key[e] & 0xFFFFu] : -1;
    else oi[e] = ok ? (int32_t)(0xFFFFu - (key[e] & 0xFFFFu)) : -1;
    ov[e] = ok ? unord16(key[e] >> 16) : (uint16_t)0;
  }
  // 16-byte stores when the thread's whole run lies inside the row and rows are
  // 16-byte aligned (k % 8 == 0); the rest element by element
  if (E % 8 == 0 && k % 8 == 0 && E * t + E <= k) {
#pragma unroll
    for (int e = 0; e < E; e += 4)
      *reinterpret_cast<int4*>(iout + E * t + e) = make_int4(oi[e], oi[e + 1], oi[e + 2], oi[e + 3]);
    if (vout)
#pragma unroll
      for (int e = 0; e < E; e += 8)
        *reinterpret_cast<uint4*>(vout + E * t + e) =
            make_uint4(ov[e] | ((uint32_t)ov[e + 1] << 16), ov[e + 2] | ((uint32_t)ov[e + 3] << 16),
                       ov[e + 4] | ((uint32_t)ov[e + 5] << 16), ov[e + 6] | ((uint32_t)ov[e + 7] << 16));
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int i = E * t + e;
      if (i < k) {
        iout[i] = oi[e];
        if (vout) vout[i] = ov[e];
      }
    }
  }
}

}  // namespace
}  // namespace dsa

template <bool WIDE>
static hipError_t launch_topk_e(const LiTopkArgs& a, int e, unsigned rows, hipStream_t s) {
  const dim3 grid(rows), block(dsa::TPB);
  if (e <= 1) hipLaunchKernelGGL((dsa::li_topk_kernel<1, WIDE>), grid, block, 0, s, a);
  else if (e <= 2) hipLaunchKernelGGL((dsa::li_topk_kernel<2, WIDE>), grid, block, 0, s, a);
  else if (e <= 4) hipLaunchKernelGGL((dsa::li_topk_kernel<4, WIDE>), grid, block, 0, s, a);
  else if (e <= 8) hipLaunchKernelGGL((dsa::li_topk_kernel<8, WIDE>), grid, block, 0, s, a);
  else if (e <= 16) hipLaunchKernelGGL((dsa::li_topk_kernel<16, WIDE>), grid, block, 0, s, a);
  else if (e <= 32) hipLaunchKernelGGL((dsa::li_topk_kernel<32, WIDE>), grid, block, 0, s, a);
  else hipLaunchKernelGGL((dsa::li_topk_kernel<64, WIDE>), grid, block, 0, s, a);
  return hipGetLastError();
}

hipError_t launch_li_topk(const LiTopkArgs& a, hipStream_t s) {
  const int64_t rows = (int64_t)a.total_rows * a.n2;
  if (rows <= 0) return hipSuccess;
  const int e = (a.k + dsa::TPB - 1) / dsa::TPB;
  return a.s2 > 65536 ? launch_topk_e<true>(a, e, (unsigned)rows, s) : launch_topk_e<false>(a, e, (unsigned)rows, s);
}
