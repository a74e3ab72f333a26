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
//      VGPRs as packed pairs (rows longer than 8192 entries are streamed from
//      memory instead, in chunks of 8192). Waves holding no entry of the row skip
//      the per-entry loops below.
//   2. L > k: a 2048-bin LDS histogram of u >> 5, scanned from the top bin, gives
//      the bin holding the k-th largest key and the number of keys above that bin.
//   3. Order-preserving compaction: keys of higher bins go, in index order, to
//      positions p < k as (u << 16 | x), p from a block exclusive scan of the
//      per-thread counts (packed 16-bit counting on the key pairs); the keys of the
//      bin go to a candidate list, among which a 32-bin histogram of the low 5 bits
//      finds the exact threshold T and how many keys equal to T to take; those
//      follow, also in index order. Rows of up to 65536 entries carry
//      x = 0xFFFF - index; longer rows (WIDE) carry x = p and keep the 32-bit index
//      in a second LDS array at p (p, like the index, increases along the row).
//      Rows with L <= k take every entry at its own index.
//   4. A stable LSD radix sort ascending on v = umax - u (score descending; umax
//      and umin bound the selected keys), 4-bit digits, over only the digits that
//      umax - umin spans. Each thread counts the digits of its keys with LDS atomics
//      on its own 16-bit counters (the returned value is the key's rank among the
//      thread's earlier keys of that digit), one block scan turns the per-thread
//      counts into scatter offsets. Stability preserves the index order of equal
//      scores, which is exactly the golden's tie rule.
//   5. One pass writes the indices and 16-bit values in rank order.
// The selection histogram and the sort's counters share one LDS array (they are
// never live together), so a work-group needs ~16 KB and more of them fit a CU.
#include "dsa_common.hpp"

namespace dsa {
namespace {

constexpr int TPB = 256;
constexpr int RPT = 32;                 // row entries per thread held in VGPRs
constexpr int ROW_CACHED = TPB * RPT;   // 8192

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

// Block-wide exclusive scan (wave scans with DPP, one LDS exchange); also returns the total.
// One barrier: every caller has a block barrier between the previous reads of `red` (the
// last scan's) and this call (the compaction and candidate scans follow the barriers of
// the bin pick and of the candidate resolution, each sort pass's scan the pass's count
// barrier), so the words are free to overwrite.
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t* red, uint32_t* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t x = wave_incl_sum(v);
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

typedef short i16x2 __attribute__((ext_vector_type(2)));

// ord16 of both 16-bit halves of w (see ord16), four VALU ops for the pair: a half h
// becomes h ^ (sign-extended sign | 0x8000) plus its sign bit, i.e. h | 0x8000 when
// positive and ~h + 1 = 0x10000 - h when negative (-0 lands on +0's 0x8000). No half
// carries into the next: a negative half gives at most 0x7FFF + 1.
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t ord16x2(uint32_t w) {
  const uint32_t s = __builtin_bit_cast(uint32_t, __builtin_bit_cast(i16x2, w) >> (i16x2){15, 15});
  const uint32_t sb = __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, w) >> (u16x2){15, 15});
  return (w ^ (s | 0x80008000u)) + sb;
}

// Per 16-bit half of the packed keys w: 1 if the key is above c (c in both halves of
// cc), else 0 -- a saturating packed subtraction and a packed minimum with 1.
__device__ __forceinline__ uint32_t pk_above(uint32_t w, uint32_t cc) {
  uint32_t d;
  asm("v_pk_sub_u16 %0, %1, %2 clamp\n\tv_pk_min_u16 %0, %0, %3" : "=&v"(d) : "v"(w), "s"(cc), "s"(0x00010001u));
  return d;
}
// sum of the two 16-bit halves of packed counters (each at most 0x7FFF)
__device__ __forceinline__ uint32_t pk_hsum(uint32_t c) { return (c & 0xFFFFu) + (c >> 16); }
// packed 16-bit unsigned max, min and wrapping subtraction (v_pk_max_u16, v_pk_min_u16, v_pk_sub_u16)
__device__ __forceinline__ uint32_t pk_max(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2, a), __builtin_bit_cast(u16x2, b)));
}
__device__ __forceinline__ uint32_t pk_min(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_min(__builtin_bit_cast(u16x2, a), __builtin_bit_cast(u16x2, b)));
}
__device__ __forceinline__ uint32_t pk_sub(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, a) - __builtin_bit_cast(u16x2, b));
}
// Stores v at *p and advances p by one word in place, for the active lanes of a divergent
// branch. Written in C++ (`*p++ = v`) the compiler computes the new pointer into another
// register before the store and copies it back: two VALU ops per store instead of one.
typedef __attribute__((address_space(3))) uint32_t lds_u32;
__device__ __forceinline__ void lds_push(lds_u32*& p, uint32_t v) {
  *p = v;
  asm volatile("v_add_u32 %0, 4, %0" : "+v"(p));
}
// key e of a thread's packed pairs (w[e / 2], low half = even e)
__device__ __forceinline__ uint32_t kh(const uint32_t* w, int e) { return (e & 1) ? w[e >> 1] >> 16 : w[e >> 1] & 0xFFFFu; }

// Keys [base + 32t, +32) of the row as packed ord16 pairs; entries at or past L are 0
// (below every real key). Threads whose entries all lie past L load nothing.
__device__ __forceinline__ void load_keys(const uint16_t* row, int L, int base, uint32_t (&w)[RPT / 2]) {
  const int i0 = base + threadIdx.x * RPT;
  if (i0 + RPT <= L) {
#pragma unroll
    for (int c = 0; c < RPT / 8; ++c) {
      const uint4 v = ldg16(row + i0 + c * 8);
      w[c * 4 + 0] = ord16x2(v.x);
      w[c * 4 + 1] = ord16x2(v.y);
      w[c * 4 + 2] = ord16x2(v.z);
      w[c * 4 + 3] = ord16x2(v.w);
    }
  } else if (i0 < L) {
#pragma unroll
    for (int e = 0; e < RPT; e += 2) {
      const uint32_t lo = (i0 + e < L) ? ord16(row[i0 + e]) : 0u;
      const uint32_t hi = (i0 + e + 1 < L) ? ord16(row[i0 + e + 1]) : 0u;
      w[e >> 1] = lo | (hi << 16);
    }
  } else {
#pragma unroll
    for (int e = 0; e < RPT / 2; ++e) w[e] = 0u;
  }
}

// Rank block of thread t in the sort: lanes l and l + 32 of a wave hold the neighbouring
// blocks 2m, 2m + 1 (m = 32 w + l), so the thread pair sharing a 32-bit counter word sits
// in different half-waves, and the 32 lanes of a half-wave reach 32 different banks.
__device__ __forceinline__ int rank_block(int t) { return (t & ~63) | ((t & 31) << 1) | ((t >> 5) & 1); }

// Stable LSD radix sort of E keys per thread (blocked: thread t holds ranks
// [E b, E b + E), b = rank_block(t)), ascending on the upper 16 bits, over passes
// [0, npass) (4 bits each, from the low bits up). `cnt` holds 16 x TPB 16-bit counters in
// [digit][block] order; a thread counts its keys with LDS atomics on its own counter (a
// 32-bit add of 1 or 1 << 16 on the word it shares with the thread of the neighbouring
// block), whose returned value is the key's rank among the thread's earlier keys of that
// digit.
// Entries at ranks >= n are padding whose digits are all 15 (and whose values are
// never read back): they stay behind every real key in each pass, so they affect no
// real key's position, and a wave holding padding only neither counts nor moves it
// (the ranks past the active waves' slots are then left stale).
template <int E>
__device__ __forceinline__ void radix_sort_asc16(uint32_t (&key)[E], int npass, int n, uint32_t* sbuf,
                                                 uint16_t* cnt, uint32_t* red) {
  const int t = threadIdx.x, tb = rank_block(t);
  const bool act = (int)__builtin_amdgcn_readfirstlane(t >> 6) * 64 * E < n;
  const uint32_t inc = (tb & 1) ? 0x10000u : 1u, hsh = (tb & 1) ? 16u : 0u;
  uint32_t* cw = reinterpret_cast<uint32_t*>(cnt) + (tb >> 1);   // digit 0's word of this thread pair
#pragma unroll 1
  for (int pass = 0; pass < npass; ++pass) {
    const int shift = 16 + 4 * pass;
    // the pair's counter words, digits 8 (tb & 1) .. +8 by this thread: both threads of a
    // pair sit in one wave, whose LDS operations run in order, and no other wave touches
    // these words before the barrier below (the last pass's scatter read only its own)
#pragma unroll
    for (int d = 0; d < 8; ++d) cw[(8 * (tb & 1) + d) * (TPB / 2)] = 0u;
    uint32_t lrank[E];
    if (act)
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const uint32_t d = __builtin_amdgcn_ubfe(key[e], shift, 4);
        lrank[e] = (atomicAdd(cw + d * (TPB / 2), inc) >> hsh) & 0xFFFFu;
      }
    __syncthreads();
    // exclusive scan over cnt in [digit][block] order: thread t scans entries 16t..16t+15
    const uint4 q0 = *reinterpret_cast<const uint4*>(cnt + t * 16);
    const uint4 q1 = *reinterpret_cast<const uint4*>(cnt + t * 16 + 8);
    const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    uint32_t s = 0;   // both halves at once: a half sums at most 8 counts of at most E keys
#pragma unroll
    for (int j = 0; j < 8; ++j) s += w[j];
    s = (s & 0xFFFFu) + (s >> 16);
    uint32_t tot;
    uint32_t run = block_excl_scan(s, red, &tot);   // offset of this thread's first entry
    uint32_t o[8];   // running offsets, re-derived from the counts (no second array live across the scan)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t lo = run;
      run += w[j] & 0xFFFFu;
      o[j] = lo | (run << 16);
      run += w[j] >> 16;
    }
    *reinterpret_cast<uint4*>(cnt + t * 16) = make_uint4(o[0], o[1], o[2], o[3]);
    *reinterpret_cast<uint4*>(cnt + t * 16 + 8) = make_uint4(o[4], o[5], o[6], o[7]);
    __syncthreads();
    if (act)
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int d = __builtin_amdgcn_ubfe(key[e], shift, 4);
        // byte offset (offset + rank) * 4 in one op (the compiler shifts both terms)
        uint32_t bo;
        asm("v_add_lshl_u32 %0, %1, %2, 2" : "=v"(bo) : "v"((uint32_t)cnt[d * TPB + tb]), "v"(lrank[e]));
        *reinterpret_cast<lds_u32*>((__attribute__((address_space(3))) uint8_t*)sbuf + bo) = key[e];
      }
    __syncthreads();
    if (act)
#pragma unroll
      for (int e = 0; e < E; ++e) key[e] = sbuf[E * tb + e];
    // the next pass writes cnt (read above, before the barrier) and sbuf (after two barriers)
  }
}

// Block-wide exclusive scan of v together with the maxima of m1 and m2 (every thread
// gets the scan total and both maxima): one LDS exchange for the three. LEAD: a barrier
// first, for callers whose threads may still be reading `red` from an earlier scan (a
// caller's first scan of the row needs none). M2 = false: m2 is unused (max2 gets 0).
template <bool LEAD = true, bool M2 = true>
__device__ __forceinline__ uint32_t block_scan_max2(uint32_t v, uint32_t m1, uint32_t m2, uint32_t* red,
                                                    uint32_t* total, uint32_t* max1, uint32_t* max2) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t x = wave_incl_sum(v);
  m1 = wave_incl_max(m1);   // lane 63: the wave's maximum
  if constexpr (M2) m2 = wave_incl_max(m2);
  if constexpr (LEAD) __syncthreads();
  if (lane == 63) {
    red[wave] = x;
    red[TPB / 64 + wave] = m1;
    red[2 * (TPB / 64) + wave] = m2;
  }
  __syncthreads();
  uint32_t off = 0, tot = 0, a = 0, b = 0;
#pragma unroll
  for (int w = 0; w < TPB / 64; ++w) {
    off += (w < wave) ? red[w] : 0u;
    tot += red[w];
    a = max(a, red[TPB / 64 + w]);
    if constexpr (M2) b = max(b, red[2 * (TPB / 64) + w]);
  }
  *total = tot;
  *max1 = a;
  *max2 = b;
  return off + x - v;
}

// SHORT: rows of at most ROW_CACHED entries (s2 <= 8192), held in registers in one chunk;
// the chunked paths for longer rows are compiled out. Short rows with k <= 2048 are
// compiled for eight waves per SIMD (64 VGPRs, 96 SGPRs: more SGPR spills to VGPR lanes,
// which cost less than the latency an eighth work-group per CU hides). At eight waves per
// SIMD the VALU issues for about two thirds of the kernel's time; LDS bank conflicts and
// the chain of block barriers take most of the rest.
template <int E, bool WIDE, bool SHORT = false>
__global__ __launch_bounds__(TPB) __attribute__((amdgpu_waves_per_eu(SHORT && E <= 8 ? 8 : 1, 8)))
void li_topk_kernel(LiTopkArgs a) {
  static_assert(!(SHORT && WIDE), "short rows use 16-bit indices");
  static_assert(E * TPB <= 65536, "compacted positions are 16-bit");
  constexpr int HWORDS = 2048;         // selection histogram (u >> 5), then the candidate list
  constexpr int CWORDS = 16 * TPB / 2;   // sort counters (16-bit)
  __shared__ __attribute__((aligned(16))) uint32_t sbuf[E * TPB];
  __shared__ int32_t sidx[WIDE ? E * TPB : 1];   // WIDE: row index of compacted position p
  __shared__ __attribute__((aligned(16))) uint32_t work[HWORDS > CWORDS ? HWORDS : CWORDS];
  __shared__ uint32_t red[3 * (TPB / 64)];
  __shared__ uint32_t pick[3];
  __shared__ uint32_t chist[32];
  uint32_t* hist = work;
  uint16_t* cnt = reinterpret_cast<uint16_t*>(work);

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
  const int nchunks = SHORT ? 1 : (L + ROW_CACHED - 1) / ROW_CACHED;
  uint32_t w[RPT / 2];   // the thread's keys, packed pairs
  if (nchunks == 1) load_keys(row, L, 0, w);
  // one chunk: whether this wave holds any entry of the row (the per-entry loops of the
  // others are skipped: every key they hold is 0)
  const bool wv = nchunks > 1 || __builtin_amdgcn_readfirstlane(t >> 6) * 64 * RPT < L;
  uint32_t T = 0;  // keys > T are all taken; keys == T up to `need`
  uint32_t need = 0xFFFFFFFFu;
  uint32_t umin = 0, umax = 0xFFFFu;   // bounds of the selected keys (the sort's pass range)
  bool compacted = false;
  if (L > k) {
    // 2048-bin histogram of u >> 5, scanned from the top bin: bin b holds the k-th
    // largest key, `above` keys lie in higher bins (all taken)
#pragma unroll
    for (int i = 0; i < 8; ++i) hist[t * 8 + i] = 0;
    __syncthreads();
#pragma unroll 1
    for (int ch = 0; ch < nchunks; ++ch) {
      if (nchunks > 1) load_keys(row, L, ch * ROW_CACHED, w);
      // every key of a thread holding part of the row is counted, with no per-key test:
      // the padding past L of the one thread straddling L lands in bin 0 and is taken
      // out below (threads wholly past L count nothing, so bin 0 sees no pile-up)
      if (ch * ROW_CACHED + t * RPT < L)
#pragma unroll
        for (int i = 0; i < RPT / 2; ++i) {   // the bins of both keys of a pair, straight from the word
          const uint32_t x = w[i];
          atomicAdd(&hist[(x >> 5) & 0x7FFu], 1u);
          atomicAdd(&hist[x >> 21], 1u);
        }
    }
    __syncthreads();
    uint32_t h[8];   // thread t: bins 2047 - 8t - j, j < 8 (the scan runs from the top)
    {
      const uint4 lo4 = *reinterpret_cast<const uint4*>(&hist[2040 - 8 * t]);
      const uint4 hi4 = *reinterpret_cast<const uint4*>(&hist[2044 - 8 * t]);
      h[0] = hi4.w; h[1] = hi4.z; h[2] = hi4.y; h[3] = hi4.x;
      h[4] = lo4.w; h[5] = lo4.z; h[6] = lo4.y; h[7] = lo4.x;
    }
    if (t == TPB - 1) h[7] -= (uint32_t)(-L & (RPT - 1));   // bin 0: the padding counted above
    uint32_t hs = 0, top1 = 0;   // top1: highest non-empty bin + 1 (0: none)
#pragma unroll
    for (int j = 7; j >= 0; --j) {
      hs += h[j];
      top1 = h[j] ? (uint32_t)(2048 - 8 * t - j) : top1;
    }
    uint32_t tot, btop1, unused;
    uint32_t cum = block_scan_max2<false, false>(hs, top1, 0u, red, &tot, &btop1, &unused);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (cum < (uint32_t)k && cum + h[j] >= (uint32_t)k) {
        pick[0] = 2047 - 8 * t - j;
        pick[1] = cum;
        pick[2] = h[j];
      }
      cum += h[j];
    }
    __syncthreads();
    const uint32_t bin = pick[0], above = pick[1], nc = pick[2];
    umax = ((btop1 - 1) << 5) | 31u;
    const uint32_t need_c = (uint32_t)k - above;   // keys of bin `bin` to take
    // the k-th largest within bin `bin`: a 32-bin histogram of the low 5 bits of its
    // keys, scanned from the top by wave 0; sets T and `need`
    auto resolve = [&](auto&& count_keys) {
      if (t < 32) chist[t] = 0;
      __syncthreads();
      count_keys();
      __syncthreads();
      if (t < 64) {   // wave 0, all lanes active (DPP)
        const uint32_t hh = t < 32 ? chist[31 - t] : 0u;
        const uint32_t incl = wave_incl_sum(hh);
        if (t < 32 && incl - hh < need_c && incl >= need_c) {
          pick[0] = 31 - t;
          pick[1] = incl - hh;
        }
      }
      __syncthreads();
      T = (bin << 5) | pick[0];
      need = need_c - pick[1];
    };
    if (!WIDE && nchunks == 1 && nc <= (uint32_t)HWORDS) {
      // one pass over the row: keys of higher bins go to sbuf[0, above) in index order,
      // the keys of bin `bin` to a candidate list (the same key << 16 | 0xFFFF - index,
      // index order) in the histogram's place; T is then found among the candidates only, and the
      // selected ones follow in sbuf, in index order. The two groups hold different
      // keys, so their relative order is irrelevant to the stable sort.
      uint32_t* cand = work;
      const int i0 = t * RPT;
      // cg: keys of higher bins (>= (bin + 1) << 5); cc: nonzero keys of bin `bin` (keys
      // >= max(bin << 5, 1), minus cg), counted per packed pair (per-half sums <= 16)
      const uint32_t g1 = ((bin + 1) << 5) - 1, b1 = bin == 0 ? 0u : (bin << 5) - 1;
      uint32_t ag = 0, ab = 0;
      if (wv)
#pragma unroll
        for (int i = 0; i < RPT / 2; ++i) {
          ag += pk_above(w[i], g1 * 0x10001u);
          ab += pk_above(w[i], b1 * 0x10001u);
        }
      const uint32_t cg = pk_hsum(ag), cc = pk_hsum(ab) - cg;
      uint32_t tot1;
      const uint32_t pgc = block_excl_scan((cg << 16) | cc, red, &tot1);
      lds_u32* ps = (lds_u32*)(sbuf + (pgc >> 16));
      lds_u32* pcd = (lds_u32*)(cand + (pgc & 0xFFFFu));
      const uint32_t xb = 0xFFFFu - (uint32_t)i0;
      if (wv)
#pragma unroll
        for (int e = 0; e < RPT; ++e) {
          // key << 16 | (0xFFFF - index), built from the key's half in two ops (the empty
          // asm keeps the compiler from splitting xb - e around the shift); the compares
          // read the key in its half
          uint32_t x = xb - e;
          asm("" : "+v"(x));
          const uint32_t v = (e & 1) ? ((w[e >> 1] & 0xFFFF0000u) | x) : ((w[e >> 1] << 16) | x);
          const uint32_t ue = kh(w, e);
          const bool hi = ue > g1;
          if (hi) lds_push(ps, v);               // a higher bin
          if (ue > b1 && !hi) lds_push(pcd, v);  // bin `bin`, nonzero
        }
      // candidates [c0, c1) of this thread (at most 8: nc <= 2048; the loops stop at the
      // block-uniform m, typically 1 or 2)
      const uint32_t m = (nc + TPB - 1) / TPB, c0 = min((uint32_t)t * m, nc), c1 = min(c0 + m, nc);
      resolve([&] {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if (j >= (int)m) break;
          if (c0 + j < c1) atomicAdd(&chist[(cand[c0 + j] >> 16) & 31u], 1u);
        }
      });
      uint32_t cv[8];
      uint32_t g2 = 0, e2 = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (j >= (int)m) break;
        cv[j] = c0 + j < c1 ? cand[c0 + j] : 0u;
        g2 += (c0 + j < c1 && (cv[j] >> 16) > T) ? 1u : 0u;
        e2 += (c0 + j < c1 && (cv[j] >> 16) == T) ? 1u : 0u;
      }
      uint32_t tot2;
      const uint32_t pge = block_excl_scan((g2 << 16) | e2, red, &tot2);
      uint32_t qg = above + (pge >> 16), qe = pge & 0xFFFFu;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (j >= (int)m) break;
        if (c0 + j >= c1) continue;
        const uint32_t key16 = cv[j] >> 16, x = cv[j] & 0xFFFFu;
        if (key16 > T) {
          sbuf[qg + (qe < need ? qe : need)] = (key16 << 16) | x;
          ++qg;
        } else if (key16 == T) {
          if (qe < need) sbuf[qg + qe] = (key16 << 16) | x;
          ++qe;
        }
      }
      compacted = true;
    } else {   // rows longer than 8192 or a crowded bin: one more pass over the row
      resolve([&] {
#pragma unroll 1
        for (int ch = 0; ch < nchunks; ++ch) {
          if (nchunks > 1) load_keys(row, L, ch * ROW_CACHED, w);
#pragma unroll
          for (int e = 0; e < RPT; ++e)
            if (kh(w, e) != 0u && (kh(w, e) >> 5) == bin) atomicAdd(&chist[kh(w, e) & 31u], 1u);
        }
      });
    }
    umin = T;
  }
  if constexpr (SHORT) {
    if (L <= k) {
      // every visible entry is taken, at its own index (the keys past L are 0 and are
      // not written); the largest key and the smallest nonzero one bound the sort's
      // passes, as in the general path below
      const int i0 = t * RPT;
      uint32_t mx2 = 0, mn2 = 0xFFFFFFFFu;   // per half: largest key, smallest key - 1 (0 wraps to 0xFFFF)
#pragma unroll
      for (int i = 0; i < RPT / 2; ++i) {
        mx2 = pk_max(mx2, w[i]);
        mn2 = pk_min(mn2, pk_sub(w[i], 0x00010001u));
      }
      const uint32_t mx = max(mx2 & 0xFFFFu, mx2 >> 16), mnm1 = min(mn2 & 0xFFFFu, mn2 >> 16);
      const uint32_t mninv = mnm1 == 0xFFFFu ? 0u : 0xFFFEu - mnm1;   // 0xFFFF - smallest nonzero key
      if (i0 + RPT <= L) {
        const uint32_t xb = 0xFFFFu - (uint32_t)i0;
#pragma unroll
        for (int c = 0; c < RPT / 4; ++c) {   // entries 4c .. 4c + 3: words 2c, 2c + 1
          const uint32_t w0 = w[2 * c], w1 = w[2 * c + 1];
          *reinterpret_cast<uint4*>(&sbuf[i0 + 4 * c]) =
              make_uint4((w0 << 16) | (xb - 4 * c), (w0 & 0xFFFF0000u) | (xb - 4 * c - 1),
                         (w1 << 16) | (xb - 4 * c - 2), (w1 & 0xFFFF0000u) | (xb - 4 * c - 3));
        }
      } else if (i0 < L) {   // the one thread holding the row's end
#pragma unroll
        for (int e = 0; e < RPT; ++e)
          if (i0 + e < L) sbuf[i0 + e] = (kh(w, e) << 16) | (0xFFFFu - (uint32_t)(i0 + e));
      }
      uint32_t tot, cmx, cmn;
      block_scan_max2<false>(0u, mx, mninv, red, &tot, &cmx, &cmn);
      umax = cmx;
      umin = 0xFFFFu - cmn;
      compacted = true;
    }
  }
  if (!compacted) {
    // positions: selected-before = greater-before + min(ties-before, need); one scan of
    // (greater << 16 | ties) per chunk (a chunk holds at most 8192 of each), which also
    // gives the largest and smallest key (the sort's pass range when every key is taken)
    uint32_t run_g = 0, run_e = 0;  // totals of previous chunks
    uint32_t kmax = 0, kmin_inv = 0;   // max of u, max of 0xFFFF - u over nonzero keys
#pragma unroll 1
    for (int ch = 0; ch < nchunks; ++ch) {
      if (nchunks > 1) load_keys(row, L, ch * ROW_CACHED, w);
      const int i0 = ch * ROW_CACHED + t * RPT;
      uint32_t cg = 0, ce = 0, mx = 0, mn = 0;
#pragma unroll
      for (int e = 0; e < RPT; ++e) {
        const uint32_t ue = kh(w, e);
        cg += ue > T ? 1u : 0u;
        ce += (ue == T && T != 0) ? 1u : 0u;
        mx = max(mx, ue);
        mn = ue != 0u ? max(mn, 0xFFFFu - ue) : mn;
      }
      uint32_t tot, cmx, cmn;
      const uint32_t pgs = block_scan_max2((cg << 16) | ce, mx, mn, red, &tot, &cmx, &cmn);
      kmax = max(kmax, cmx);
      kmin_inv = max(kmin_inv, cmn);
      uint32_t pg = (pgs >> 16) + run_g;
      uint32_t pe = (pgs & 0xFFFFu) + run_e;
#pragma unroll
      for (int e = 0; e < RPT; ++e) {
        const uint32_t ue = kh(w, e);
        // x: the index (rows up to 65536) or the position, whose index goes to sidx
        auto put = [&](uint32_t p) {
          if constexpr (WIDE) {
            sbuf[p] = (ue << 16) | p;
            sidx[p] = i0 + e;
          } else {
            sbuf[p] = (ue << 16) | (0xFFFFu - (uint32_t)(i0 + e));
          }
        };
        if (ue > T) {
          put(pg + (pe < need ? pe : need));
          ++pg;
        } else if (ue == T && T != 0) {
          if (pe < need) put(pg + pe);
          ++pe;
        }
      }
      run_g += tot >> 16;
      run_e += tot & 0xFFFFu;
    }
    if (L <= k) {
      umax = kmax;
      umin = 0xFFFFu - kmin_inv;
    }
  }
  for (int i = nout + t; i < E * TPB; i += TPB) sbuf[i] = 0u;  // pads sort last
  __syncthreads();

  // ---- stable radix sort of the selected keys, then write in rank order. The sort runs
  // ascending on v = umax - key (score descending), over the 4-bit digits that
  // umax - umin spans; the padding entries (key 0) take v = 16^npass - 1, the largest
  // value those digits hold, and being last in the input they stay last among equals.
  const uint32_t urange = umax > umin ? umax - umin : 0u;
  const int npass = urange == 0 ? 0 : (35 - __builtin_clz(urange)) / 4;
  const uint32_t vmax = (1u << (4 * npass)) - 1u;
  uint32_t key[E];
  const int tb = rank_block(t);   // the thread's rank block in the sort and the output
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const uint32_t x = sbuf[E * tb + e];
    key[e] = (min(umax - (x >> 16), vmax) << 16) | (x & 0xFFFFu);
  }
  radix_sort_asc16<E>(key, npass, nout, sbuf, cnt, red);
  // ranks E tb .. E tb + E - 1 of thread t: their index (or -1) and 16-bit value (or 0).
  // A run of 8 ranks inside the row's output, all below nout (the usual case): indices
  // 0xFFFF - x, values unord16(umax - v) computed on packed pairs.
  if (!WIDE && E % 8 == 0 && k % 8 == 0 && E * tb + E <= nout) {
    const uint32_t um2x = (umax ^ 0x8000u) * 0x10001u;   // umax - 0x8000 in both halves
#pragma unroll
    for (int e = 0; e < E; e += 8) {
      uint32_t pv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // upper halves (v) of keys e + 2j and e + 2j + 1; the key is umax - v per half
        const uint32_t vv = __builtin_amdgcn_perm(key[e + 2 * j + 1], key[e + 2 * j], 0x07060302u);
        // unord16 per half from d = key - 0x8000 (signed: the value's magnitude, negated
        // for a negative value): |d| with d's sign bit
        const i16x2 d = __builtin_bit_cast(i16x2, pk_sub(um2x, vv));
        const uint32_t ad = __builtin_bit_cast(uint32_t, __builtin_elementwise_max(d, (i16x2){0, 0} - d));
        pv[j] = ad | (__builtin_bit_cast(uint32_t, d) & 0x80008000u);
      }
      *reinterpret_cast<int4*>(iout + E * tb + e) =
          make_int4((int)(~key[e] & 0xFFFFu), (int)(~key[e + 1] & 0xFFFFu), (int)(~key[e + 2] & 0xFFFFu),
                    (int)(~key[e + 3] & 0xFFFFu));
      *reinterpret_cast<int4*>(iout + E * tb + e + 4) =
          make_int4((int)(~key[e + 4] & 0xFFFFu), (int)(~key[e + 5] & 0xFFFFu), (int)(~key[e + 6] & 0xFFFFu),
                    (int)(~key[e + 7] & 0xFFFFu));
      if (vout) *reinterpret_cast<uint4*>(vout + E * tb + e) = make_uint4(pv[0], pv[1], pv[2], pv[3]);
    }
    return;
  }
  int32_t oi[E];
  uint16_t ov[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const bool ok = E * tb + e < nout;
    if constexpr (WIDE) oi[e] = ok ? sidx[key[e] & 0xFFFFu] : -1;
    else oi[e] = ok ? (int32_t)(0xFFFFu - (key[e] & 0xFFFFu)) : -1;
    ov[e] = ok ? unord16(umax - (key[e] >> 16)) : (uint16_t)0;
  }
  // 16-byte stores when the thread's whole run lies inside the row and rows are
  // 16-byte aligned (k % 8 == 0); the rest element by element
  if (E % 8 == 0 && k % 8 == 0 && E * tb + E <= k) {
#pragma unroll
    for (int e = 0; e < E; e += 4)
      *reinterpret_cast<int4*>(iout + E * tb + e) = make_int4(oi[e], oi[e + 1], oi[e + 2], oi[e + 3]);
    if (vout)
#pragma unroll
      for (int e = 0; e < E; e += 8)
        *reinterpret_cast<uint4*>(vout + E * tb + e) =
            make_uint4(ov[e] | ((uint32_t)ov[e + 1] << 16), ov[e + 2] | ((uint32_t)ov[e + 3] << 16),
                       ov[e + 4] | ((uint32_t)ov[e + 5] << 16), ov[e + 6] | ((uint32_t)ov[e + 7] << 16));
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int i = E * tb + e;
      if (i < k) {
        iout[i] = oi[e];
        if (vout) vout[i] = ov[e];
      }
    }
  }
}

// ---------------------------------------------------------------- sparse_count > LI_TOPK_MAX_K
// Rows whose top-k does not fit the LDS sort (k > 16384): one 1024-thread work-group
// per score row sorts every visible entry in global scratch (two buffers of S2 entries
// per row, caller-provided) and writes the first min(L, k). Entries are
// (v << 32 | index), v = umax - key (score descending), written in index order; a
// stable LSD radix sort on v (4-bit digits, over the digits umax - umin spans) then
// keeps the index order of equal scores, the golden's tie rule. Thread t owns the
// contiguous input range [t C, t C + C) of each pass; its per-digit counters and, after
// the block scan in (digit, thread) order, its scatter offsets are LDS words of its own.
constexpr int BIG_TPB = 1024;

__device__ __forceinline__ uint32_t big_block_scan(uint32_t v, uint32_t* red, uint32_t* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t x = wave_incl_sum(v);
  __syncthreads();
  if (lane == 63) red[wave] = x;
  __syncthreads();
  uint32_t off = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < BIG_TPB / 64; ++w) {
    off += (w < wave) ? red[w] : 0u;
    tot += red[w];
  }
  *total = tot;
  return off + x - v;
}

__global__ __launch_bounds__(BIG_TPB) void li_topk_big_kernel(LiTopkArgs a, uint64_t* ws) {
  __shared__ uint32_t cnt[16 * BIG_TPB];   // [digit][thread]: counts, then scatter offsets
  __shared__ uint32_t red[2 * (BIG_TPB / 64)];
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
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  if (nout == 0) {
    for (int i = t; i < k; i += BIG_TPB) {
      iout[i] = -1;
      if (vout) vout[i] = 0;
    }
    return;
  }
  uint64_t* src = ws + (int64_t)sr * 2 * a.s2;
  uint64_t* dst = src + a.s2;
  // the range of the row's keys: largest key, and 0xFFFF - the smallest
  uint32_t mx = 0, mi = 0;
  for (int i = t; i < L; i += BIG_TPB) {
    const uint32_t u = ord16(row[i]);
    mx = max(mx, u);
    mi = max(mi, 0xFFFFu - u);
  }
  mx = wave_incl_max(mx);
  mi = wave_incl_max(mi);
  if (lane == 63) {
    red[wave] = mx;
    red[BIG_TPB / 64 + wave] = mi;
  }
  __syncthreads();
  uint32_t umax = 0, uminv = 0;
#pragma unroll
  for (int w = 0; w < BIG_TPB / 64; ++w) {
    umax = max(umax, red[w]);
    uminv = max(uminv, red[BIG_TPB / 64 + w]);
  }
  const uint32_t urange = umax - (0xFFFFu - uminv);
  const int npass = urange == 0 ? 0 : (35 - __builtin_clz(urange)) / 4;
  for (int i = t; i < L; i += BIG_TPB) src[i] = ((uint64_t)(umax - ord16(row[i])) << 32) | (uint32_t)i;
  __syncthreads();   // (also: every read of red above is done before the scans reuse it)
  const int C = (L + BIG_TPB - 1) / BIG_TPB;
  const int c0 = min(t * C, L), c1 = min(c0 + C, L);
  for (int pass = 0; pass < npass; ++pass) {
    const int shift = 32 + 4 * pass;
#pragma unroll
    for (int d = 0; d < 16; ++d) cnt[d * BIG_TPB + t] = 0;
    for (int i = c0; i < c1; ++i) ++cnt[(int)((src[i] >> shift) & 15u) * BIG_TPB + t];
    __syncthreads();
    // exclusive scan in (digit, thread) order: thread t scans words 16t .. 16t + 15
    uint32_t w[16], s = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      w[j] = cnt[16 * t + j];
      s += w[j];
    }
    uint32_t tot;
    uint32_t run = big_block_scan(s, red, &tot);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      cnt[16 * t + j] = run;
      run += w[j];
    }
    __syncthreads();
    for (int i = c0; i < c1; ++i) {
      const uint64_t e = src[i];
      const int d = (int)((e >> shift) & 15u);
      dst[cnt[d * BIG_TPB + t]++] = e;
    }
    __syncthreads();   // the pass's output is complete (and visible) before the next reads it
    uint64_t* tmp = src;
    src = dst;
    dst = tmp;
  }
  for (int i = t; i < k; i += BIG_TPB) {
    if (i < nout) {
      const uint64_t e = src[i];
      iout[i] = (int32_t)(uint32_t)e;
      if (vout) vout[i] = unord16(umax - (uint32_t)(e >> 32));
    } else {
      iout[i] = -1;
      if (vout) vout[i] = 0;
    }
  }
}

}  // namespace
}  // namespace dsa

template <bool WIDE, bool SHORT>
static hipError_t launch_topk_e(const LiTopkArgs& a, int e, unsigned rows, hipStream_t s) {
  const dim3 grid(rows), block(dsa::TPB);
  if (e <= 1) hipLaunchKernelGGL((dsa::li_topk_kernel<1, WIDE, SHORT>), grid, block, 0, s, a);
  else if (e <= 2) hipLaunchKernelGGL((dsa::li_topk_kernel<2, WIDE, SHORT>), grid, block, 0, s, a);
  else if (e <= 4) hipLaunchKernelGGL((dsa::li_topk_kernel<4, WIDE, SHORT>), grid, block, 0, s, a);
  else if (e <= 8) hipLaunchKernelGGL((dsa::li_topk_kernel<8, WIDE, SHORT>), grid, block, 0, s, a);
  else if (e <= 16) hipLaunchKernelGGL((dsa::li_topk_kernel<16, WIDE, SHORT>), grid, block, 0, s, a);
  else if (e <= 32) hipLaunchKernelGGL((dsa::li_topk_kernel<32, WIDE, SHORT>), grid, block, 0, s, a);
  else hipLaunchKernelGGL((dsa::li_topk_kernel<64, WIDE, SHORT>), grid, block, 0, s, a);
  return hipGetLastError();
}

size_t li_topk_workspace_bytes(int total_rows, int n2, int s2, int k) {
  if (k <= LI_TOPK_MAX_K || total_rows <= 0 || n2 <= 0 || s2 <= 0) return 0;
  return (size_t)total_rows * n2 * 2 * s2 * sizeof(uint64_t);
}

hipError_t launch_li_topk_big(const LiTopkArgs& a, void* ws, hipStream_t s) {
  const int64_t rows = (int64_t)a.total_rows * a.n2;
  if (rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(dsa::li_topk_big_kernel, dim3((unsigned)rows), dim3(dsa::BIG_TPB), 0, s, a,
                     reinterpret_cast<uint64_t*>(ws));
  return hipGetLastError();
}

hipError_t launch_li_topk(const LiTopkArgs& a, hipStream_t s) {
  const int64_t rows = (int64_t)a.total_rows * a.n2;
  if (rows <= 0) return hipSuccess;
  const int e = (a.k + dsa::TPB - 1) / dsa::TPB;
  if (a.s2 > 65536) return launch_topk_e<true, false>(a, e, (unsigned)rows, s);
  if (a.s2 > dsa::ROW_CACHED) return launch_topk_e<false, false>(a, e, (unsigned)rows, s);
  return launch_topk_e<false, true>(a, e, (unsigned)rows, s);   // every visible row fits the registers
}
