// Sparse flash attention forward (MLA-absorb, N2 = 1) for gfx950.
//
// Semantics: sparse_flash_attention_numpy.py:38-160 (the golden) with the
// layouts of sparse_flash_attention_triton.py:1353-1450.
//
// Kernels:
//  1. sfa_tokens_kernel (sfa_tokens1_kernel when sparse_block_size == 1: one
//     wave per row) -- one work-group per packed query row: applies the
//     row-skip rules and the golden's gatherKV scan (first
//     min(count, ceil(threshold/bs)) ids, stop at the first -1, expand id to
//     [id*bs, min(id*bs+bs, act_k, threshold))) and writes the row's token list
//     as PHYSICAL key rows (key_start offset, or the PA block-table lookup; a -1
//     block or an out-of-range row becomes the zero row). Replaces the
//     reference's host-side _expand_block_indices / _pa_to_bsnd (:1012-1051)
//     and its masked loads (:392-398).
//  2. sfa_attn_kernel -- one work-group (4 waves, one per SIMD) per (query row,
//     KV split) covering all (up to 128) heads, so every gathered KV row is
//     fetched once per row:
//       * tokens are processed in tiles of 32; a tile's [D | Dr] rows are
//         gathered with direct-to-LDS 16-byte loads (no VGPR staging) into a
//         ring of three LDS buffers, two tiles ahead of the one being computed;
//         the token ids travel the same ordered path (a 4-slot LDS ring filled
//         four tiles ahead), the loads are spread over the S^T MFMA chain and
//         the per-tile barriers are LDS-only, so nothing drains the gathers in
//         flight and one partial vmcnt wait per tile retires the oldest tile;
//       * S^T = K Q^T on v_mfma_f32_32x32x16 with tokens as M and 32 heads per
//         wave as N (Q^T resident in VGPRs): a lane then holds 16 tokens of one
//         head, so the softmax row max is in-lane plus one lane swap;
//       * online softmax in fp32 with lazy rescaling: the exponent reference
//         m_used only moves when a tile's max exceeds it by more than TAU
//         (natural-log units; 40 for bf16, 8 for fp16 so that P = exp(s - m_used)
//         stays finite once packed to fp16), so O is rarely rescaled; the true
//         max is tracked for softmax_max;
//       * P (io dtype) goes to LDS as [head][token]; each wave then owns a
//         D/4-column slice of O[128 heads, D] and accumulates it transposed,
//         O^T += V^T P^T, on v_mfma_f32_32x32x16, the V^T operand read with
//         ds_read_b64_tr_b16 straight from the gathered rows (value = key), so
//         a lane holds one head and runs of four consecutive columns;
//       * O stays in registers; the epilogue divides by the row sum and writes
//         16-byte rows (with several KV splits the normalised partial goes out
//         in the io dtype).
//  3. sfa_merge_kernel -- merges KV-split partials (log-sum-exp weights) of the
//     rows whose tokens span several splits. With KV splits and
//     sparse_block_size 1 (decode) each split lists its own tokens inside
//     sfa_attn_kernel, so a decode call is two launches.
// Unlike the reference (sparse_flash_attention_triton.py:509-525) the fp32
// accumulator never round-trips through HBM for unsplit rows.
#include <climits>
#include <mutex>
#include <type_traits>

#include "dsa_common.hpp"

namespace dsa {
namespace {

constexpr int DR = 64;
constexpr float LOG2E = 1.4426950408889634f;

struct RowInfo {
  int b, s1, aq, ak, threshold;
  bool active;
};

__device__ __forceinline__ RowInfo row_info(const SfaArgs& a, int r) {
  RowInfo ri;
  ri.b = batch_of_row(a.row_start, a.batch, r);
  ri.s1 = r - a.row_start[ri.b];
  ri.aq = a.act_q[ri.b];
  ri.ak = a.act_k[ri.b];
  ri.active = ri.s1 < ri.aq;
  if (a.sparse_mode != 0 && ri.s1 < ri.aq - ri.ak) ri.active = false;  // numpy_golden:125-126
  ri.threshold = a.sparse_mode == 0 ? ri.ak : ri.ak - ri.aq + ri.s1 + 1;
  if (ri.threshold <= 0) ri.active = false;                             // numpy_golden:131-132
  return ri;
}

// ---------------------------------------------------------------- workspace
// The zero KV row comes first; it must be zero when the workspace is first used
// (no launch writes anything else there, the token-list kernels rewrite zeros).
struct Ws {
  uint16_t* zero;    // one zero KV row: 512 + Dr elements
  int32_t* counts;   // [rows]   token-list length of the row
  int32_t* tokens;   // [rows, tstride]
  int tstride;       // token-list row stride: cap rounded up to a whole 32-token tile
  uint16_t* part_o;  // [rows, splits, N1, D]   O_s / l_s in the io dtype (splits > 1)
  float* part_s;     // [rows, splits, N1, 3]   m_used, m_true, l
};

__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

__host__ __device__ inline Ws ws_layout(void* base, int rows, int cap, int n1, int d, int splits,
                                        size_t* total) {
  char* p = reinterpret_cast<char*>(base);
  size_t off = 0;
  Ws w;
  w.tstride = (cap + 31) & ~31;
  w.zero = reinterpret_cast<uint16_t*>(p + off);
  off += align256((size_t)(512 + DR) * 2);
  w.counts = reinterpret_cast<int32_t*>(p + off);
  off += align256((size_t)rows * 4);
  w.tokens = reinterpret_cast<int32_t*>(p + off);
  off += align256((size_t)rows * w.tstride * 4);
  w.part_o = reinterpret_cast<uint16_t*>(p + off);
  w.part_s = nullptr;
  if (splits > 1) {
    off += align256((size_t)rows * splits * n1 * d * 2);
    w.part_s = reinterpret_cast<float*>(p + off);
    off += align256((size_t)rows * splits * n1 * 3 * 4);
  }
  if (total) *total = off;
  return w;
}

// ---------------------------------------------------------------- kernel 1
constexpr int TOK_TPB = 256;
constexpr int TOK_PER = 8;                       // ids per thread per pass
constexpr int TOK_CHUNK = TOK_TPB * TOK_PER;     // ids per pass

// Work-group (TOK_TPB threads) reductions through LDS. LDS_ONLY barriers order
// the LDS traffic alone, so global loads in flight (a prefetch) are not drained.
template <bool LDS_ONLY = false>
__device__ __forceinline__ void red_barrier() {
  if constexpr (LDS_ONLY) lds_barrier(); else __syncthreads();
}

template <bool LDS_ONLY = false>
__device__ __forceinline__ int block_min_i(int v, int* red) {
  v = wave_incl_min_i32(v);   // lane 63: the wave's minimum (DPP, no LDS round trips)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  red_barrier<LDS_ONLY>();
  if (lane == 63) red[wave] = v;
  red_barrier<LDS_ONLY>();
  int m = red[0];
#pragma unroll
  for (int w = 1; w < TOK_TPB / 64; ++w) m = min(m, red[w]);
  return __builtin_amdgcn_readfirstlane(m);   // uniform; read from LDS, so not provably so
}

template <bool LDS_ONLY = false>
__device__ __forceinline__ int block_sum_i(int v, int* red) {
  v = (int)wave_incl_sum((uint32_t)v);   // lane 63: the wave's sum
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  red_barrier<LDS_ONLY>();
  if (lane == 63) red[wave] = v;
  red_barrier<LDS_ONLY>();
  int t = 0;
#pragma unroll
  for (int w = 0; w < TOK_TPB / 64; ++w) t += red[w];
  return __builtin_amdgcn_readfirstlane(t);
}

// exclusive block scan of v; *tot receives the block total
template <bool LDS_ONLY = false>
__device__ __forceinline__ int block_excl_scan_i(int v, int* red, int* tot) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int x = (int)wave_incl_sum((uint32_t)v);
  red_barrier<LDS_ONLY>();
  if (lane == 63) red[wave] = x;
  red_barrier<LDS_ONLY>();
  int off = 0, t = 0;
#pragma unroll
  for (int w = 0; w < TOK_TPB / 64; ++w) {
    off += w < wave ? red[w] : 0;
    t += red[w];
  }
  *tot = __builtin_amdgcn_readfirstlane(t);
  return off + x - v;
}

// One work-group per packed query row. Pass c covers ids [c*2048, c*2048+2048):
// thread t holds ids 8t..8t+7 of the pass in registers (one load each, issued
// together), the first -1 is found with a block min, per-thread token counts
// are scanned to output positions, and every page-table lookup of the thread is
// issued before its stores.
__global__ __launch_bounds__(TOK_TPB) void sfa_tokens_kernel(SfaArgs a, int cap, Ws ws) {
  __shared__ int red[TOK_TPB / 64];
  const int r = blockIdx.x;
  const int tid = threadIdx.x;
  if (r == 0)
    for (int i = tid; i < 512 + DR; i += TOK_TPB) ws.zero[i] = 0;
  const RowInfo ri = row_info(a, r);
  if (!ri.active) {
    if (tid == 0) ws.counts[r] = 0;
    return;
  }
  const int bs = a.sbs;
  const int64_t ceil_blocks = ((int64_t)ri.threshold + bs - 1) / bs;
  const int nscan0 = (int)((int64_t)a.topk < ceil_blocks ? a.topk : ceil_blocks);
  const int32_t* ids = a.sidx + (int64_t)r * a.topk;
  const int end_lim = ri.ak < ri.threshold ? ri.ak : ri.threshold;
  int32_t* out = ws.tokens + (int64_t)r * ws.tstride;
  // page of token t: shift and mask for power-of-two page sizes (32-bit division otherwise)
  const bool pow2 = a.block_table && (a.page_bs & (a.page_bs - 1)) == 0;
  const int pshift = pow2 ? __builtin_ctz((unsigned)a.page_bs) : 0;
  auto phys_row = [&](int64_t t) -> int32_t {
    int64_t p;
    if (a.block_table) {
      const int bi = pow2 ? (int)(t >> pshift) : (int)((uint64_t)t / (unsigned)a.page_bs);
      const int within = (int)(t - (int64_t)bi * a.page_bs);
      const int blk = bi < a.max_blocks ? a.block_table[(int64_t)ri.b * a.max_blocks + bi] : -1;
      p = blk < 0 ? -1 : (int64_t)blk * a.page_bs + within;
    } else {
      p = t < a.s2 ? (int64_t)a.key_start[ri.b] + t : -1;
    }
    return (p >= 0 && p < a.key_rows) ? (int32_t)p : -1;
  };
  int base = 0;   // tokens written by earlier passes
  for (int c0 = 0; c0 < nscan0; c0 += TOK_CHUNK) {
    const int g0 = c0 + tid * TOK_PER;
    int v[TOK_PER];
#pragma unroll
    for (int j = 0; j < TOK_PER; ++j) v[j] = g0 + j < nscan0 ? ids[g0 + j] : -2;  // -2: past the scan
    int fneg = INT_MAX;
#pragma unroll
    for (int j = TOK_PER - 1; j >= 0; --j) fneg = v[j] == -1 ? g0 + j : fneg;
    fneg = block_min_i(fneg, red);   // the scan stops at the first -1 (only -1 is defined to stop it)
    int cnt[TOK_PER], my = 0;
#pragma unroll
    for (int j = 0; j < TOK_PER; ++j) {
      int n = 0;
      if (g0 + j < fneg && v[j] >= 0) {   // other negative ids are skipped
        const int64_t begin = (int64_t)v[j] * bs;
        if (begin < ri.threshold) {
          const int64_t e = begin + bs < end_lim ? begin + bs : end_lim;
          n = e > begin ? (int)(e - begin) : 0;
        }
      }
      cnt[j] = n;
      my += n;
    }
    int tot;
    int pos = base + block_excl_scan_i(my, red, &tot);
    if (bs == 1) {
      int32_t pr[TOK_PER];
#pragma unroll
      for (int j = 0; j < TOK_PER; ++j) pr[j] = cnt[j] ? phys_row(v[j]) : 0;
#pragma unroll
      for (int j = 0; j < TOK_PER; ++j)
        if (cnt[j]) out[pos++] = pr[j];
    } else {
#pragma unroll 1
      for (int j = 0; j < TOK_PER; ++j)
        for (int k = 0; k < cnt[j]; ++k) out[pos++] = phys_row((int64_t)v[j] * bs + k);
    }
    base += tot;
    if (fneg != INT_MAX) break;
  }
  if (tid == 0) ws.counts[r] = base;
}

// sparse_block_size == 1 (every id is one token): one wave per packed query row,
// TOK1_ROWS rows per work-group, no block-level synchronisation. Pass c covers ids
// [c*2048, c*2048+2048): lane l loads the 16-byte groups i*64 + l (i < 8) of the
// pass, i.e. ids 4(i*64 + l) .. +3; the first -1 (wave min) ends the scan. Ids are
// kept in id order: a valid id's output slot is the number of valid ids before it,
// counted with one ballot + mbcnt per (group row i, position j in the group).
constexpr int TOK1_ROWS = 4;

__global__ __launch_bounds__(64 * TOK1_ROWS) void sfa_tokens1_kernel(SfaArgs a, int cap, Ws ws) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * TOK1_ROWS + (threadIdx.x >> 6);
  if (blockIdx.x == 0)
    for (int i = threadIdx.x; i < 512 + DR; i += 64 * TOK1_ROWS) ws.zero[i] = 0;
  if (r >= a.total_rows) return;
  const RowInfo ri = row_info(a, r);
  if (!ri.active) {
    if (lane == 0) ws.counts[r] = 0;
    return;
  }
  const int nscan0 = a.topk < ri.threshold ? a.topk : ri.threshold;
  const int32_t* ids = a.sidx + (int64_t)r * a.topk;
  const int end_lim = ri.ak < ri.threshold ? ri.ak : ri.threshold;
  int32_t* out = ws.tokens + (int64_t)r * ws.tstride;
  const bool vec = (a.topk & 3) == 0;   // 16-byte aligned rows
  // page of token t: shift and mask for power-of-two page sizes (32-bit division otherwise)
  const bool pow2 = a.block_table && (a.page_bs & (a.page_bs - 1)) == 0;
  const int pshift = pow2 ? __builtin_ctz((unsigned)a.page_bs) : 0;
  auto phys_row = [&](int t) -> int32_t {
    int64_t p;
    if (a.block_table) {
      const int bi = pow2 ? t >> pshift : (int)((unsigned)t / (unsigned)a.page_bs);
      const int within = t - bi * a.page_bs;
      const int blk = bi < a.max_blocks ? a.block_table[(int64_t)ri.b * a.max_blocks + bi] : -1;
      p = blk < 0 ? -1 : (int64_t)blk * a.page_bs + within;
    } else {
      p = t < a.s2 ? (int64_t)a.key_start[ri.b] + t : -1;
    }
    return (p >= 0 && p < a.key_rows) ? (int32_t)p : -1;
  };
  const uint32_t lo_mask = lane < 32 ? (1u << lane) - 1u : 0xFFFFFFFFu;
  const uint32_t hi_mask = lane < 32 ? 0u : (lane == 32 ? 0u : (1u << (lane - 32)) - 1u);
  auto below = [&](uint64_t m) {   // set bits of m in lanes below this one
    return __builtin_popcount((uint32_t)m & lo_mask) + __builtin_popcount((uint32_t)(m >> 32) & hi_mask);
  };
  int base = 0;   // tokens written by earlier passes
  for (int c0 = 0; c0 < nscan0; c0 += 2048) {
    int v[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int g = c0 + (i * 64 + lane) * 4;
      if (vec && g + 3 < nscan0) {
        const int4 x = *reinterpret_cast<const int4*>(ids + g);
        v[i][0] = x.x; v[i][1] = x.y; v[i][2] = x.z; v[i][3] = x.w;
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) v[i][j] = g + j < nscan0 ? ids[g + j] : -2;   // -2: past the scan
      }
    }
    int fneg = INT_MAX;
#pragma unroll
    for (int i = 7; i >= 0; --i)
#pragma unroll
      for (int j = 3; j >= 0; --j) fneg = v[i][j] == -1 ? c0 + (i * 64 + lane) * 4 + j : fneg;
    fneg = __builtin_amdgcn_readlane(wave_incl_min_i32(fneg), 63);   // only -1 stops the scan
    bool ok[8][4];
    int32_t pr[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int pos = c0 + (i * 64 + lane) * 4 + j;
        ok[i][j] = pos < fneg && v[i][j] >= 0 && v[i][j] < end_lim;   // other negative ids are skipped
        pr[i][j] = ok[i][j] ? phys_row(v[i][j]) : 0;                  // every lookup issued before the stores
      }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      int off = base, mine = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint64_t m = __ballot(ok[i][j]);
        off += below(m);
        base += __popcll(m);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (ok[i][j]) out[off + mine++] = pr[i][j];
    }
    if (fneg != INT_MAX) break;
  }
  if (lane == 0) ws.counts[r] = base;
}

// ---------------------------------------------------------------- split-local token lists
// Loads a KV split issues at the very start of the attention kernel when it lists
// its own tokens (sparse_block_size 1): ids [8t, 8t+8) of the row's first 2048
// (-2 past sparse_count), this thread's share of the batch count (batches
// b = t, t + 256, ... whose rows end at or before r) and, for b = t, the batch's
// first row and lengths (broadcast once the batch is known).
struct TokPrefetch {
  int v[TOK_PER];
  int bcnt;
  int rs0, aq, ak;
};

__device__ __forceinline__ TokPrefetch tok_prefetch(const SfaArgs& a, int r) {
  TokPrefetch p;
  const int32_t* ids = a.sidx + (int64_t)r * a.topk;
  const int g0 = threadIdx.x * TOK_PER;
  if ((a.topk & 3) == 0 && g0 + TOK_PER <= a.topk) {   // 16-byte aligned, whole
    const int4 x0 = *reinterpret_cast<const int4*>(ids + g0);
    const int4 x1 = *reinterpret_cast<const int4*>(ids + g0 + 4);
    p.v[0] = x0.x; p.v[1] = x0.y; p.v[2] = x0.z; p.v[3] = x0.w;
    p.v[4] = x1.x; p.v[5] = x1.y; p.v[6] = x1.z; p.v[7] = x1.w;
  } else {
#pragma unroll
    for (int j = 0; j < TOK_PER; ++j) p.v[j] = g0 + j < a.topk ? ids[g0 + j] : -2;
  }
  const int b = threadIdx.x;
  const bool own = b < a.batch;
  p.rs0 = own ? a.row_start[b] : 0;
  p.aq = own ? a.act_q[b] : 0;
  p.ak = own ? a.act_k[b] : 0;
  p.bcnt = own && a.row_start[b + 1] <= r ? 1 : 0;
  for (int bb = b + TOK_TPB; bb < a.batch; bb += TOK_TPB) p.bcnt += a.row_start[bb + 1] <= r ? 1 : 0;
  return p;
}

// The part of row r's token list that KV split sp (of `splits`) processes, for
// sparse_block_size 1, built by the split's own work-group (TOK_TPB threads): the
// golden's gatherKV scan (numpy golden :44-49 -- positions below
// min(count, threshold), up to the first -1, ids in [0, min(act_k, threshold)))
// numbers the row's tokens in id order; the split owns numbers
// [sp*per, min(sp*per + per, n)), per = ceil(ceil(n / splits) / 32) * 32 (the
// split rule of the attention kernel), and writes their physical rows to the
// row's token list at those positions. Returns n (0 for a skipped row); the batch
// is the count of batches ending at or before r (rows past the last batch map to
// it). A scan longer than one 2048-id pass counts first, then numbers. Barriers
// are LDS-only: loads issued before the call stay in flight. The split's first
// four tiles are also written to the LDS id ring s_ids; issue_q() (the kernel's Q
// loads) is called right after the block-table lookups are issued, once.
template <typename IssueQ>
__device__ int split_token_list(const SfaArgs& a, int r, int sp, int splits, const Ws& ws, int* red,
                                const TokPrefetch& pre, int32_t (*s_ids)[32], IssueQ&& issue_q) {
  const int tid = threadIdx.x;
  RowInfo ri;
  const int nb = block_sum_i<true>(pre.bcnt, red);
  ri.b = nb < a.batch ? nb : a.batch - 1;
  if (a.batch <= TOK_TPB) {   // the batch's thread broadcasts what it prefetched
    if (tid == ri.b) {
      red[4] = pre.rs0;
      red[5] = pre.aq;
      red[6] = pre.ak;
    }
    lds_barrier();
    ri.s1 = r - __builtin_amdgcn_readfirstlane(red[4]);
    ri.aq = __builtin_amdgcn_readfirstlane(red[5]);
    ri.ak = __builtin_amdgcn_readfirstlane(red[6]);
  } else {
    ri.s1 = r - a.row_start[ri.b];
    ri.aq = a.act_q[ri.b];
    ri.ak = a.act_k[ri.b];
  }
  ri.active = ri.s1 < ri.aq;
  if (a.sparse_mode != 0 && ri.s1 < ri.aq - ri.ak) ri.active = false;  // numpy_golden:125-126
  ri.threshold = a.sparse_mode == 0 ? ri.ak : ri.ak - ri.aq + ri.s1 + 1;
  if (ri.threshold <= 0) ri.active = false;                             // numpy_golden:131-132
  bool q_issued = false;
  if (!ri.active) {
    issue_q();
    return 0;
  }
  const int nscan0 = a.topk < ri.threshold ? a.topk : ri.threshold;
  const int end_lim = ri.ak < ri.threshold ? ri.ak : ri.threshold;
  const int32_t* ids = a.sidx + (int64_t)r * a.topk;
  int32_t* out = ws.tokens + (int64_t)r * ws.tstride;
  const bool pow2 = a.block_table && (a.page_bs & (a.page_bs - 1)) == 0;
  const int pshift = pow2 ? __builtin_ctz((unsigned)a.page_bs) : 0;
  auto phys_row = [&](int t) -> int32_t {
    int64_t p;
    if (a.block_table) {
      const int bi = pow2 ? t >> pshift : (int)((unsigned)t / (unsigned)a.page_bs);
      const int within = t - bi * a.page_bs;
      const int blk = bi < a.max_blocks ? a.block_table[(int64_t)ri.b * a.max_blocks + bi] : -1;
      p = blk < 0 ? -1 : (int64_t)blk * a.page_bs + within;
    } else {
      p = t < a.s2 ? (int64_t)a.key_start[ri.b] + t : -1;
    }
    return (p >= 0 && p < a.key_rows) ? (int32_t)p : -1;
  };
  // one pass: ids 8t..8t+7 of [c0, c0 + 2048) per thread (pass 0 from the
  // prefetch), validity, the first -1
  auto pass = [&](int c0, int (&v)[TOK_PER], bool (&ok)[TOK_PER], int& fneg) {
    const int g0 = c0 + tid * TOK_PER;
#pragma unroll
    for (int j = 0; j < TOK_PER; ++j)
      v[j] = g0 + j < nscan0 ? (c0 == 0 ? pre.v[j] : ids[g0 + j]) : -2;   // -2: past the scan
    fneg = INT_MAX;
#pragma unroll
    for (int j = TOK_PER - 1; j >= 0; --j) fneg = v[j] == -1 ? g0 + j : fneg;
    fneg = block_min_i<true>(fneg, red);   // only -1 stops the scan
#pragma unroll
    for (int j = 0; j < TOK_PER; ++j) ok[j] = g0 + j < fneg && v[j] >= 0 && v[j] < end_lim;
  };
  int v[TOK_PER];
  bool ok[TOK_PER];
  int fneg, n = 0;
  const bool multi = nscan0 > TOK_CHUNK;
  if (multi)
    for (int c0 = 0; c0 < nscan0; c0 += TOK_CHUNK) {
      pass(c0, v, ok, fneg);
      int my = 0;
#pragma unroll
      for (int j = 0; j < TOK_PER; ++j) my += ok[j];
      n += block_sum_i<true>(my, red);
      if (fneg != INT_MAX) break;
    }
  int base = 0;
  for (int c0 = 0; c0 < nscan0; c0 += TOK_CHUNK) {
    pass(c0, v, ok, fneg);
    int my = 0;
#pragma unroll
    for (int j = 0; j < TOK_PER; ++j) my += ok[j];
    int tot;
    const int pos = base + block_excl_scan_i<true>(my, red, &tot);
    if (!multi) n = tot;
    const int per = ((n + splits - 1) / splits + 31) / 32 * 32;
    const int t_beg = sp * per;
    const int t_end = t_beg + per < n ? t_beg + per : n;
    // this thread's valid ids are numbered pos, pos+1, ... in id order
    int32_t pr[TOK_PER];
    bool mine[TOK_PER];
    int q = pos;
#pragma unroll
    for (int j = 0; j < TOK_PER; ++j) {
      mine[j] = ok[j] && q >= t_beg && q < t_end;
      pr[j] = mine[j] ? phys_row(v[j]) : 0;   // every lookup issued before the stores
      q += ok[j] ? 1 : 0;
    }
    if (!q_issued) {   // Q after the lookups, so waiting for these does not wait for Q
      issue_q();
      q_issued = true;
    }
    // every position goes to the row's token list (the ring copies of the tiles
    // past the split's end re-read its last tile from there); the split's first 4
    // tiles also go straight to the id ring (slot t: tile t; slots past the split's
    // last tile repeat it, as the ring copies do)
    const int ntl = (t_end - t_beg + 31) / 32;
    q = pos;
#pragma unroll
    for (int j = 0; j < TOK_PER; ++j) {
      if (mine[j]) {
        const int pl = q - t_beg;
        out[q] = pr[j];
        if (pl < 4 * 32) {
          s_ids[pl >> 5][pl & 31] = pr[j];
          if ((pl >> 5) == ntl - 1)
            for (int t = ntl; t < 4; ++t) s_ids[t][pl & 31] = pr[j];
        }
      }
      q += ok[j] ? 1 : 0;
    }
    base += tot;
    if (fneg != INT_MAX || base >= t_end) break;
  }
  if (!q_issued) issue_q();
  return n;
}

// ---------------------------------------------------------------- kernel 3
// Merge of the KV-split partials of the rows whose tokens span several splits
// (the attention kernel writes single-split and skipped rows itself). Work-group
// (row, blockIdx.y) covers units u = (head u / (D/8), columns 8 (u % (D/8)) ..+8),
// one unit per thread for at most MS splits, every partial load issued before any
// is used. Split s left O_s / l_s (io dtype) and (m_used_s, m_true_s, l_s); per
// head M = max m_used_s, w_s = l_s 2^((m_used_s - M) log2 e),
// out = sum_s w_s (O_s / l_s) / sum_s w_s; softmax_max / sum as for an unsplit row.
template <int IO, int D, int MS>
__global__ __launch_bounds__(256) void sfa_merge_kernel(SfaArgs a, int splits, Ws ws) {
  constexpr int MERGE_MAX_SPLITS = MS, MU = 1;   // units per thread (more were slower: fewer waves in flight)
  const int r = blockIdx.x;
  const int n1 = a.n1;
  constexpr int CH = D / 8;
  const int units = n1 * CH;
  const float* ps = ws.part_s + (int64_t)r * splits * n1 * 3;
  const uint16_t* po = ws.part_o + (int64_t)r * splits * n1 * D;
  uint16_t* out = reinterpret_cast<uint16_t*>(a.out) + (int64_t)r * n1 * D;
  const int u0 = blockIdx.y * 256 * MU + threadIdx.x;
  // every split's partial and statistics are requested before the row's token count
  // (which says how many splits hold tokens) has arrived: one memory round trip instead
  // of two; the entries of splits past the row's tokens are in bounds and never used
  uint4 v[MU][MERGE_MAX_SPLITS];
  float sm_u[MU][MERGE_MAX_SPLITS], sm_t[MU][MERGE_MAX_SPLITS], sm_l[MU][MERGE_MAX_SPLITS];
  static_assert(CH % 64 == 0 || 64 % CH == 0, "a wave's units cover whole heads or divide one");
#pragma unroll
  for (int k = 0; k < MU; ++k) {
    const int u = u0 + k * 256;
    const int uc = u < units ? u : units - 1;
    // D >= 512: one head per wave, so its statistics are scalar loads
    const int hw = CH >= 64 ? __builtin_amdgcn_readfirstlane(uc / CH) : uc / CH;
#pragma unroll
    for (int sp = 0; sp < MERGE_MAX_SPLITS; ++sp)
      if (sp < splits) {
        v[k][sp] = ldg16(po + ((int64_t)sp * n1 + uc / CH) * D + (uc % CH) * 8);
        const float* q = ps + ((int64_t)sp * n1 + hw) * 3;
        sm_u[k][sp] = q[0];
        sm_t[k][sp] = q[1];
        sm_l[k][sp] = q[2];
      }
  }
  const int ntok_all = ws.counts[r];
  const int per = ((ntok_all + splits - 1) / splits + 31) / 32 * 32;
  const int nact = ntok_all > 0 ? (ntok_all + per - 1) / per : 0;
  if (nact <= 1) return;
#pragma unroll
  for (int k = 0; k < MU; ++k) {
    const int u = u0 + k * 256;
    if (u >= units) continue;
    const int h = u / CH;
    float M = -INFINITY, mt = -INFINITY;
#pragma unroll
    for (int sp = 0; sp < MERGE_MAX_SPLITS; ++sp)
      if (sp < nact) {
        M = fmaxf(M, sm_u[k][sp]);
        mt = fmaxf(mt, sm_t[k][sp]);
      }
    float w[MERGE_MAX_SPLITS];
    float L = 0.f;
#pragma unroll
    for (int sp = 0; sp < MERGE_MAX_SPLITS; ++sp) {
      w[sp] = sp < nact ? sm_l[k][sp] * exp2f((sm_u[k][sp] - M) * LOG2E) : 0.f;
      L += w[sp];
    }
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int sp = 0; sp < MERGE_MAX_SPLITS; ++sp)
      if (sp < nact) {
        const uint32_t x[4] = {v[k][sp].x, v[k][sp].y, v[k][sp].z, v[k][sp].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc[2 * j] += w[sp] * to_f32<IO>((uint16_t)(x[j] & 0xFFFFu));
          acc[2 * j + 1] += w[sp] * to_f32<IO>((uint16_t)(x[j] >> 16));
        }
      }
    const float il = 1.f / L;   // L >= l of the split holding the max > 0
    stg16(out + (int64_t)h * D + (u % CH) * 8,
          make_uint4(pack2<IO>(acc[0] * il, acc[1] * il), pack2<IO>(acc[2] * il, acc[3] * il),
                     pack2<IO>(acc[4] * il, acc[5] * il), pack2<IO>(acc[6] * il, acc[7] * il)));
    if (u % CH == 0 && a.sm_max) {
      a.sm_max[(int64_t)r * n1 + h] = mt;
      a.sm_sum[(int64_t)r * n1 + h] = L * exp2f((M - mt) * LOG2E);
    }
  }
}

// ---------------------------------------------------------------- kernel 2
constexpr int NWV = 4;      // waves per work-group (one per SIMD)
constexpr int BN = 32;      // tokens per tile
constexpr int NBUF = 3;     // gather ring: tile t read, t+1 and t+2 in flight
constexpr int PP = BN + 8;  // P tile pitch (elements)
constexpr int QRP = DR + 8; // Q-rope LDS pitch (elements): 144-byte rows, conflict-free 16-byte reads
// Lazy-rescale threshold (natural units): the exponent reference m_used only
// moves when a tile's max exceeds it by more than TAU, so every P = exp(x - m_used)
// of a tile is at most e^TAU and O is rarely rescaled. P is packed to the io dtype
// before the PV product, so e^TAU must be finite there: bf16 has fp32's exponent
// range (e^40 ~ 2.4e17), fp16 overflows past 65504 ~ e^11.09, so fp16 moves the
// reference at 8 nats (P <= e^8 ~ 2981).
template <int IO> constexpr float lazy_tau() { return IO == IO_F16 ? 8.f : 40.f; }
static_assert(lazy_tau<IO_F16>() < 11.0f, "fp16 P = exp(TAU) must stay below 65504");

template <int D> struct Cfg {
  static constexpr int KS = (D + DR) / 16;      // 32x32x16 k-steps of S^T
  static constexpr int KSN = D / 16;            // of which in the nope part
  static constexpr int ROW = D * 2 + 128;       // LDS bytes reserved per gathered nope row
  static constexpr int NOPE = BN * ROW;         // bytes per nope buffer
  static constexpr int ROPE = BN * DR * 2;      // bytes per rope buffer (4 groups of 8 tokens)
  static constexpr int DW = D / NWV;            // O columns per wave
  static constexpr int NT = DW / 32;            // 32-wide N tiles per wave
  static constexpr int LANES_ROW = D / 8;       // lanes that load one nope row
  static constexpr int GPW = 8 + 1 + 1;         // direct-to-LDS loads per wave per tile (8 rows, rope, ids)
};

// Start of token t's nope row inside a buffer: rows are ROW bytes apart and
// shifted by 32*(t%4) + 16*((t/4)%2) bytes so that (a) the S^T operand reads
// (8 lanes = 8 tokens, same column) and (b) the transposed V reads (4 tokens x
// 32 bytes per 16-lane group) both land on distinct LDS banks.
template <int D> __device__ __forceinline__ int nope_off(int t) {
  return t * Cfg<D>::ROW + 32 * (t & 3) + 16 * ((t >> 2) & 1);
}
// Rope chunk c (8 elements) of token t: groups of 8 tokens, [chunk][token] order,
// which is what one direct-to-LDS instruction writes for 8 tokens.
__device__ __forceinline__ int rope_off(int t, int c) { return (t >> 3) * 1024 + (c * 8 + (t & 7)) * 16; }

// Token rows of one tile for this wave (tokens 8w..8w+7): wave-uniform rows for
// the nope gathers and, per lane, the row of token lane % 8 for the rope gather.
struct TileIdx {
  int nope[8];
  int rope;
  uint32_t zero_rows = 0;   // OFF32: nope rows (bit j: part j) whose id is out of range
};

// One of the GPW - 1 gather loads of a tile for wave w: part j < 8 copies the
// nope row of token 8w + j (one instruction, D/8 lanes), part 8 the rope chunks
// of the wave's 8 tokens (lane -> token lane%8, chunk lane/8). A physical row
// outside [0, krows) -- -1 for a missing token -- reads the zero row, so no id
// can address memory outside the key tensors.
//
// OFF32 (key tensor under 4 GiB): a nope part is the key base plus a 32-bit per-lane
// offset, one VALU op, instead of a 64-bit SGPR address and a zero-row select. Its ids
// were clamped into range (ix.zero_rows marks the rows the caller zeroes once they land).
template <int D, bool OFF32 = false>
__device__ __forceinline__ void gather_part(int j, const uint16_t* kb, const uint16_t* krb,
                                            const uint16_t* zero, int krows, const TileIdx& ix,
                                            uint8_t* nope, uint8_t* rope, int wave_u, int lane) {
  using C = Cfg<D>;
  // The empty asm statements pin the address arithmetic to this point of the caller's
  // MFMA chain: the row ids are known before the chain, and without them the compiler
  // computes every part's address up front, between the chain's first two MFMAs.
  if (j < 8) {
    int phys = ix.nope[j];   // wave-uniform: the row base goes in an SGPR pair
    asm volatile("" : "+s"(phys));
    if constexpr (OFF32) {
      if (lane < C::LANES_ROW)
        lds_dma16_sbase_untracked(kb, (uint32_t)phys * (D * 2) + lane * 16, nope + nope_off<D>(wave_u * 8 + j));
      return;
    }
    const uint16_t* src = (uint32_t)phys < (uint32_t)krows ? kb + (int64_t)phys * D : zero;
    if (lane < C::LANES_ROW) lds_dma16_sbase_untracked(src, lane * 16, nope + nope_off<D>(wave_u * 8 + j));
  } else {
    int rid = ix.rope;
    asm volatile("" : "+v"(rid));
    const uint16_t* src = (uint32_t)rid < (uint32_t)krows ? krb + (int64_t)rid * DR : zero + 512;
    lds_dma16_untracked(src + (lane >> 3) * 8, rope + wave_u * 1024);
  }
}

template <int D>
__device__ __forceinline__ void gather_tile(const uint16_t* kb, const uint16_t* krb,
                                            const uint16_t* zero, int krows, const TileIdx& ix,
                                            uint8_t* nope, uint8_t* rope, int wave_u, int lane) {
#pragma unroll
  for (int j = 0; j < 9; ++j) gather_part<D>(j, kb, krb, zero, krows, ix, nope, rope, wave_u, lane);
}

// o *= f on an accumulator element kept in an AGPR (VALU cannot read AGPRs):
// read it into one temporary VGPR, scale, write it back.
__device__ __forceinline__ float agpr_scale(float o, float f) {
  float t;
  asm volatile("v_accvgpr_read_b32 %1, %0\n\tv_mul_f32 %1, %1, %2\n\tv_accvgpr_write_b32 %0, %1"
               : "+a"(o), "=&v"(t)
               : "v"(f));
  return o;
}

// NH heads per work-group: 128 (N1 <= 128, padded), or 64 for N1 <= 64. With 128 each wave
// owns a 32-head block of S^T over the whole contraction. With 64 there are two head
// blocks, so the waves pair up: wave w computes the S^T of head block w % 2 over half w / 2
// of the contraction and the two halves are added through LDS (both waves of a pair then
// hold the same scores, and the first one writes P); the PV product and O are split over
// the D columns as for 128, at half the size.
//
// TEACH: the teacher sums of the indexer KL losses instead of attention. The S MFMAs take
// their operands the other way round (S[head, token]: a lane holds 16 heads of one token),
// each tile gives t_p[slot] = (1 / N1) sum_h exp(S scale - t_max[h]) / (t_sum[h] + 1e-8)
// (in-lane over 16 heads, one lane-half swap, then across the head blocks in LDS), and
// there is no PV product, softmax state or output.
//
// OWN (128 heads, attention): each wave also runs the PV product of its own 32 heads, over
// all D columns (O^T[D, 32 heads] in AGPRs). P never leaves the wave's registers: the
// softmax turns the S^T accumulator into the PV B operands with two lane-half swaps, so
// no wave waits for another's P, and the transposed V operands of tile t are read ahead
// during the S^T chain of tile t+1 (four times the V^T reads of the column split, at the
// LDS rate of conflict-free transposed reads). The softmax of tile t is staged over that
// chain, and the PV MFMAs of tile t follow it; one barrier per tile guards the ring.
template <int IO, int D, int NH, bool TEACH, bool OWN = false>
__global__ __launch_bounds__(NWV * 64) void sfa_attn_kernel(SfaArgs a, int cap, int splits, int fuse_tok, Ws ws) {
  using C = Cfg<D>;
  static_assert(NH == 128 || NH == 64, "heads per work-group");
  static_assert(!OWN || (NH == 128 && !TEACH), "per-wave PV: 128-head attention only");
  constexpr int MT = NH / 32;                      // 32-head blocks
  constexpr bool KSPLIT = NH == 64;                // S^T contraction split over wave pairs
  constexpr int KSH = KSPLIT ? C::KS / 2 : C::KS;  // S^T k-steps per wave
  static_assert(!KSPLIT || (C::KS % 2 == 0 && KSH <= C::KSN), "first half of the contraction is nope");
  // OWN: before the first gathers the ring is the staging area of Q^T nope (NH * D * 2
  // bytes, which may exceed the ring)
  constexpr int QSTAGE = OWN ? NH * D * 2 : 0;
  constexpr int NOPE_RAW = NBUF * C::NOPE > QSTAGE ? NBUF * C::NOPE : QSTAGE;
  __shared__ __attribute__((aligned(16))) uint8_t nope_raw[NOPE_RAW];
  uint8_t(*const nope_buf)[C::NOPE] = reinterpret_cast<uint8_t(*)[C::NOPE]>(nope_raw);
  __shared__ __attribute__((aligned(16))) uint8_t rope_buf[NBUF][C::ROPE];
  __shared__ __attribute__((aligned(16))) uint16_t pt[2][OWN ? 8 : NH * PP];   // P of tiles t (PV) and t+1 (softmax)
  __shared__ __attribute__((aligned(16))) uint16_t qrs[NH * QRP];   // Q rope of all heads
  __shared__ __attribute__((aligned(16))) int32_t s_ids[4][BN];   // token-id ring (tiles t+2 .. t+4)
  __shared__ float s_alpha[2][NH];   // O rescale factors of tiles t and t+1
  __shared__ float s_l[NH];   // 1 / row sum, per head
  __shared__ __attribute__((aligned(16))) float s_xch[KSPLIT ? NWV : 1][KSPLIT ? 16 * 64 : 4];   // S^T halves

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // rows in reverse order: under causal masks the last rows of a batch hold the most
  // tokens, so the long rows start first and short ones fill the end of the grid
  const int r = a.total_rows - 1 - (int)blockIdx.x;
  const int sp = blockIdx.y;
  const int n1 = a.n1;
  const float cpos = a.scale > 0.f ? a.scale : a.scale < 0.f ? -a.scale : 1e-30f;
  const float cl2 = cpos * LOG2E;
  // a scalar load (token-list kernel ran), waited for at its first use below
  const int ntok_pre = fuse_tok ? 0 : ws.counts[r];
  TokPrefetch pre{};
  if (fuse_tok) pre = tok_prefetch(a, r);   // requested first: the token list waits on them
  // ---- Q: Q^T (B operand of S^T, nope part) for this wave's 32 heads goes to
  // VGPRs; the Q rope of all heads is held in VGPRs (4 chunks per thread) until it
  // is written to LDS. Head indices are clamped so every wave issues the same
  // loads (padded heads are zeroed afterwards). Nothing here depends on the token
  // list: these loads are in flight while the row's token count and ids are
  // fetched (or, when the split lists its own tokens, from its block-table lookups on).
  const int kh = KSPLIT ? wave >> 1 : 0;   // this wave's half of the S^T contraction
  const int hq = (KSPLIT ? wave & 1 : wave) * 32 + (lane & 31);
  // Q^T nope fragments of this wave's k-steps kh * KSH + j (those inside the nope part)
  constexpr int QF = KSH < C::KSN ? KSH : C::KSN;
  uint4 qf[QF];
  uint4 qrv[NH * (DR / 8) / (NWV * 64)];
  float t_stat[2] = {0.f, 0.f};   // TEACH: max and sum of head threadIdx.x
  // OWN: Q^T nope goes through LDS (q_frags reads the fragments once it has landed). Wave
  // w copies its 32 heads to bytes [w * 32 D * 2, +32 D * 2) of the staging area, head
  // rows D * 2 bytes apart, with whole head rows per instruction (coalesced); the lane
  // that copies 16-byte chunk c of head h writes it at chunk c ^ (h % 16) of the row, so
  // that a fragment read (16 heads, the same chunk) lands on 16 distinct bank groups.
  constexpr int QLPR = D / 8;                                // lanes per head row
  auto q_stage = [&]() __attribute__((always_inline)) {
    const int w_u = __builtin_amdgcn_readfirstlane(wave);
    const uint16_t* q0 = reinterpret_cast<const uint16_t*>(a.q) + (int64_t)r * n1 * D;
    const int hl = lane / QLPR, c = lane % QLPR;             // head of the instruction, chunk
#pragma unroll
    for (int j = 0; j < 32 * QLPR / 64; ++j) {
      const int hb = j * (64 / QLPR);                       // the instruction's first head
      const int h = min(w_u * 32 + hb + hl, n1 - 1);
      lds_dma16_untracked(q0 + (int64_t)h * D + (c ^ ((hb + hl) & 15)) * 8,
                          nope_raw + w_u * (32 * D * 2) + hb * (D * 2));
    }
  };
  auto q_frags = [&]() __attribute__((always_inline)) {
    const uint8_t* row = nope_raw + __builtin_amdgcn_readfirstlane(wave) * (32 * D * 2) + (lane & 31) * (D * 2);
#pragma unroll
    for (int j = 0; j < QF; ++j)
      qf[j] = *reinterpret_cast<const uint4*>(row + (((2 * j + (lane >> 5)) ^ (lane & 15)) * 16));
  };
  auto issue_q = [&]() __attribute__((always_inline)) {
    if constexpr (OWN) {
      q_stage();
    } else {
      const uint16_t* qn = reinterpret_cast<const uint16_t*>(a.q) + ((int64_t)r * n1 + min(hq, n1 - 1)) * D;
#pragma unroll
      for (int j = 0; j < QF; ++j) {
        const int ks = kh * KSH + j;
        qf[j] = ldg16(qn + (ks < C::KSN ? ks : 0) * 16 + (lane >> 5) * 8);
      }
    }
#pragma unroll
    for (int j = 0; j < NH * (DR / 8) / (NWV * 64); ++j) {
      const int h = (threadIdx.x >> 3) + j * (NWV * 64 / 8), e = (threadIdx.x & 7) * 8;
      qrv[j] = ldg16(reinterpret_cast<const uint16_t*>(a.qr) + ((int64_t)r * n1 + min(h, n1 - 1)) * DR + e);
    }
    if constexpr (TEACH) {   // the row's softmax statistics, thread h < NH holds head h
      const int h = threadIdx.x < NH ? threadIdx.x : 0;
      t_stat[0] = a.t_max[(int64_t)r * n1 + min(h, n1 - 1)];
      t_stat[1] = a.t_sum[(int64_t)r * n1 + min(h, n1 - 1)];
    }
    // keeps the loads here: without it they are sunk past the branches that
    // follow and issue only once the token count has arrived
    asm volatile("" ::: "memory");
  };
  // Unsplit rows: the ids of tiles 0..3 are copied into the id ring before the token count
  // is known (one memory round trip instead of two before the first gathers). Copies stay
  // inside the row's token-list stride; ids past the row's tokens are never used for a
  // tile that is consumed (their gathers are bounded like any other).
  const bool early_ids = !fuse_tok && splits == 1;
  if (early_ids) {
    const int w_u = __builtin_amdgcn_readfirstlane(wave);
    const int32_t* toks0 = ws.tokens + (int64_t)r * ws.tstride;
#pragma unroll
    for (int t = 0; t < 4; ++t)
      if ((t + 1) * BN <= ws.tstride && lane < 2)
        lds_dma16_sbase_untracked(toks0 + t * BN + w_u * 8, lane * 16, &s_ids[t][w_u * 8]);
  }
  int ntok_all = ntok_pre;
  if (fuse_tok) {   // KV-split rows with sparse_block_size 1: this split lists its own tokens
    ntok_all = split_token_list(a, r, sp, splits, ws, reinterpret_cast<int*>(&s_alpha[0][0]), pre, s_ids,
                                issue_q);
    if (sp == 0 && threadIdx.x == 0) ws.counts[r] = ntok_all;   // for the merge kernel
  } else {
    issue_q();
  }
  // this split's token range, in whole tiles
  const int per = ((ntok_all + splits - 1) / splits + BN - 1) / BN * BN;
  const int t_beg = sp * per;
  const int t_end = (t_beg + per < ntok_all ? t_beg + per : ntok_all);
  const int ntok = t_end > t_beg ? t_end - t_beg : 0;
  const int32_t* toks = ws.tokens + (int64_t)r * ws.tstride + t_beg;
  uint16_t* out = reinterpret_cast<uint16_t*>(a.out);

  if (ntok == 0) {
    wait_vmcnt<0>();   // the Q loads above are not used on this path
    if (!TEACH && ntok_all == 0) {   // skipped row (every split sees it): zeros (out, stats), from split 0
      if (sp == 0) {
        for (int i = threadIdx.x; i < n1 * D / 8; i += NWV * 64)
          stg16(out + (int64_t)r * n1 * D + i * 8, make_uint4(0, 0, 0, 0));
        if (a.sm_max)
          for (int h = threadIdx.x; h < n1; h += NWV * 64) {
            a.sm_max[(int64_t)r * n1 + h] = 0.f;
            a.sm_sum[(int64_t)r * n1 + h] = 0.f;
          }
      }
    }   // else: a split past the row's tokens; the merge leaves it out
    return;
  }
  // KV splits holding tokens (the others returned above); with one, it writes the
  // row itself
  const int nact = (ntok_all + per - 1) / per;
  const bool direct = nact == 1;

  const uint16_t* kb = reinterpret_cast<const uint16_t*>(a.k);
  const uint16_t* krb = reinterpret_cast<const uint16_t*>(a.kr);
  const int krows = a.key_rows < INT_MAX ? (int)a.key_rows : INT_MAX;   // rows the key tensors hold
  const int ntiles = (ntok + BN - 1) / BN;

  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  // Token ids travel the same ordered path as the gathers: wave w copies ids
  // 8w..8w+7 of tile t (2 lanes x 16 B, direct-to-LDS) into ring slot t % 4, four
  // tiles ahead, just before the gathers of tile t-2; the loop-top vmcnt wait
  // that retires a tile's gathers then also covers the ids read after the
  // barrier. (Scalar loads would share lgkmcnt with the LDS reads and every LDS
  // wait would drain them.) Tiles past the end re-read the last tile, so every
  // wave issues exactly GPW loads per tile.
  auto clamp_tile = [&](int t) { return t < ntiles ? t : ntiles - 1; };
  auto ids_dma = [&](int t) {
    if (lane < 2)
      lds_dma16_sbase_untracked(toks + clamp_tile(t) * BN + wave_u * 8, lane * 16, &s_ids[t & 3][wave_u * 8]);
  };
  // ids of tile t from the ring; slots past the token list take the tile's first token
  // (off32: for gather_part<D, true>, see TileIdx::zero_rows)
  auto tile_idx = [&](int t, bool off32 = false) {
    const int tb = clamp_tile(t) * BN;
    const int nvalid = ntok - tb < BN ? ntok - tb : BN;
    const int k = wave_u * 8 + (lane & 7);
    int v = s_ids[t & 3][k];
    v = k < nvalid ? v : s_ids[t & 3][0];
    TileIdx ix;
    ix.rope = v;   // the rope gather selects the zero row itself
    if (OWN && off32) {   // nope gathers with 32-bit offsets: out-of-range ids read row 0, zeroed later
      const bool out = (uint32_t)v >= (uint32_t)krows;
      ix.zero_rows = (uint32_t)__builtin_amdgcn_ballot_w64(out) & 0xFFu;
      v = out ? 0 : v;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) ix.nope[i] = __builtin_amdgcn_readlane(v, i);
    return ix;
  };
  // ---- the ids of tiles 0..3 (copied from the token list, or already written to
  // the ring by this split's own listing); once they and Q have landed, the Q
  // rope to LDS and the first two gathers
  if (!fuse_tok) {
#pragma unroll
    for (int t = 0; t < 4; ++t)
      if (!early_ids || (t + 1) * BN > ws.tstride) ids_dma(t);
  }
  wait_vmcnt<0>();
  if constexpr (OWN) q_frags();   // this wave's own staging rows: no barrier needed
  if (hq >= n1)
#pragma unroll
    for (int j = 0; j < QF; ++j) qf[j] = make_uint4(0, 0, 0, 0);
  // The softmax works on raw scores with a positive scale cpos. A negative scale runs
  // on the negated query instead (negating 16-bit floats is exact, and so are the
  // products and their sums: -q.k exactly), so c s = |c| (-s). A zero scale becomes
  // 1e-30: scores times it round to 0 and exp of them to exactly 1, as with 0, while
  // masked slots (-inf) still give 0.
  if constexpr (!TEACH) {
    if (a.scale < 0.f) {
#pragma unroll
      for (int j = 0; j < QF; ++j) {
        qf[j].x ^= 0x80008000u;
        qf[j].y ^= 0x80008000u;
        qf[j].z ^= 0x80008000u;
        qf[j].w ^= 0x80008000u;
      }
#pragma unroll
      for (int j = 0; j < NH * (DR / 8) / (NWV * 64); ++j) {
        qrv[j].x ^= 0x80008000u;
        qrv[j].y ^= 0x80008000u;
        qrv[j].z ^= 0x80008000u;
        qrv[j].w ^= 0x80008000u;
      }
    }
  }
#pragma unroll
  for (int j = 0; j < NH * (DR / 8) / (NWV * 64); ++j) {
    const int h = (threadIdx.x >> 3) + j * (NWV * 64 / 8), e = (threadIdx.x & 7) * 8;
    *reinterpret_cast<uint4*>(qrs + h * QRP + e) = h < n1 ? qrv[j] : make_uint4(0, 0, 0, 0);
  }
  // TEACH: per-head statistics (log2 units) and the per-tile head sums share the P buffers
  float* t_mx = reinterpret_cast<float*>(&pt[0][0]);   // [NH]
  float* t_il = t_mx + NH;                              // [NH]
  float* t_tp = t_il + NH;                              // [2][NWV][BN]
  static_assert(!TEACH || (2 * NH + 2 * NWV * BN) * 4 <= (int)sizeof(pt), "teacher scratch fits the P buffers");
  if constexpr (TEACH) {
    if (threadIdx.x < NH) {
      const bool real = (int)threadIdx.x < n1;
      t_mx[threadIdx.x] = real ? t_stat[0] * LOG2E : 0.f;
      t_il[threadIdx.x] = real ? 1.f / (t_stat[1] + 1e-8f) : 0.f;   // padded heads contribute 0
    }
  }
  lds_barrier();   // (OWN: also every wave's Q^T reads of the staging area done)
  gather_tile<D>(kb, krb, ws.zero, krows, tile_idx(0), nope_buf[0], rope_buf[0], wave_u, lane);
  gather_tile<D>(kb, krb, ws.zero, krows, tile_idx(1), nope_buf[1], rope_buf[1], wave_u, lane);

  float m_used = -INFINITY, m_true = -INFINITY, l_part = 0.f;
  {
    // An AGPR operand makes the backend select the AGPR-accumulator MFMA form,
    // so O lives in AGPRs and the 256 arch VGPRs stay free for Q^T and operands.
    float agpr_hint = 0.f;
    asm volatile("" : "+a"(agpr_hint));
  }
  // O^T accumulators: [head block][32-column tile] -- all head blocks over this wave's
  // D/4 columns, or (OWN) this wave's head block over all D columns
  constexpr int OM = OWN ? 1 : MT;
  constexpr int ON = OWN ? D / 32 : C::NT;
  f32x16 o[OM][ON];
#pragma unroll
  for (int mt = 0; mt < OM; ++mt)
#pragma unroll
    for (int nt = 0; nt < ON; ++nt)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[mt][nt][i] = 0.f;

  const int tr = lane & 31, kg = lane >> 5;
  const int g16 = lane >> 4, c16 = lane & 15;
  constexpr int KQ = BN / 16;
  // Token of S^T accumulator row r = 8g + 4h + i (g < 4, h < 2, i < 4). OWN permutes the
  // rows, 16 (g/2) + 8h + 4 (g%2) + i, so that a lane's 16 scores are tokens 16 kq + 8 (lane/32)
  // + j (j < 8) of steps kq = 0, 1 -- the PV B operand's order, with no exchange between
  // lanes; otherwise row r is token r.
  auto row_tok = [](int r) { return OWN ? 16 * (r >> 4) + 8 * ((r >> 2) & 1) + 4 * ((r >> 3) & 1) + (r & 3) : r; };
  const int tk_row = row_tok(tr);   // token whose K row this lane supplies to S^T

  // ---- S^T[32 tokens, 32 heads] of tile u for this wave over k-steps [K0, K0 + KSH),
  // K0 = KH * KSH; `spread(j)` issues the loads scheduled after the chain's j-th step
  // (the next tile's gathers ride on this chain)
  auto s_tile_k = [&](int u, auto&& spread, auto khc, auto&& pre) __attribute__((always_inline)) -> f32x16 {
    constexpr int K0 = decltype(khc)::value * KSH;
    const uint8_t* nope = nope_buf[u % NBUF];
    const uint8_t* rope = rope_buf[u % NBUF];
    f32x16 sacc = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    const uint8_t* arow = nope + nope_off<D>(tk_row) + kg * 16;
    // operand loads run 4 k-steps ahead of the MFMA chain; the sched barrier
    // keeps that order (hoisting every load would cost ~4 VGPRs per k-step)
    auto a_frag = [&](int ks) -> uint4 {
      return ks < C::KSN ? *reinterpret_cast<const uint4*>(arow + ks * 32)
                         : *reinterpret_cast<const uint4*>(rope + rope_off(tk_row, (ks - C::KSN) * 2 + kg));
    };
    // the Q-rope B fragments (LDS) of the chain's rope k-steps are fetched with the
    // first operands, so the rope k-steps at the end of the chain do not wait on LDS
    // (OWN: with the K operands, as its registers are needed for the V^T operands read
    // during the chain)
    constexpr int NR = C::KS - C::KSN;
    uint4 qr[NR];
    auto qr_frag = [&](int j) -> uint4 { return *reinterpret_cast<const uint4*>(qrs + hq * QRP + j * 16 + kg * 8); };
    if constexpr (!OWN) {
#pragma unroll
      for (int j = 0; j < NR; ++j)
        if (C::KSN + j >= K0 && C::KSN + j < K0 + KSH) qr[j] = qr_frag(j);
    }
    // (OWN: five steps ahead -- LDS reads take ~200 cycles under load, four steps ~130)
    constexpr int KPF = OWN ? 5 : 4;
    uint4 af[KPF];
#pragma unroll
    for (int j = 0; j < KPF; ++j) af[j] = a_frag(K0 + j);
    pre();   // (OWN: MFMAs that cover the first operands' LDS latency)
#pragma unroll
    for (int j = 0; j < KSH; ++j) {
      const int ks = K0 + j;
      const uint4 bq = ks < C::KSN ? qf[j < QF ? j : 0] : qr[ks >= C::KSN ? ks - C::KSN : 0];
      if constexpr (TEACH) {
        sacc = Mfma<IO>::m32(bq, af[j & 3], sacc);   // S[head, token]
      } else {                                         // S^T[token, head], accumulator in VGPRs
        // the last step drains in its own statement, before the last step's loads and any VALU
        // (OWN: into fresh registers, which can be those of the loop-carried scores of the
        // previous tile -- dead by then -- so the compiler never copies an accumulator in flight)
        if (j == 0) sacc = mfma32_vacc_first<IO>(af[0], bq);
        else if (j < KSH - 1) mfma32_vacc<IO>(sacc, af[j % KPF], bq);
        else if constexpr (OWN) sacc = mfma32_vacc_last_to<IO>(sacc, af[j % KPF], bq);
        else mfma32_vacc_last<IO>(sacc, af[j % KPF], bq);
      }
      if (j + KPF < KSH) af[j % KPF] = a_frag(ks + KPF);
      if constexpr (OWN)
        if (j + KPF < KSH && ks + KPF >= C::KSN) qr[ks + KPF - C::KSN] = qr_frag(ks + KPF - C::KSN);
      spread(j);
      __builtin_amdgcn_sched_barrier(0);
    }
    return sacc;
  };
  // the full S^T of tile u for this wave's head block: one chain, or (64 heads) this
  // wave's half plus its partner's from LDS (the same sum in both waves of the pair)
  auto s_tile = [&](int u, auto&& spread) __attribute__((always_inline)) -> f32x16 {
    if constexpr (KSPLIT) {
      const int kh_u = __builtin_amdgcn_readfirstlane(kh);
      f32x16 sv = kh_u == 0 ? s_tile_k(u, spread, std::integral_constant<int, 0>{}, [] {})
                            : s_tile_k(u, spread, std::integral_constant<int, 1>{}, [] {});
      const int w_u = __builtin_amdgcn_readfirstlane(wave);
      float* mine = &s_xch[w_u][0];
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<float4*>(mine + (g * 64 + lane) * 4) =
            make_float4(sv[4 * g], sv[4 * g + 1], sv[4 * g + 2], sv[4 * g + 3]);
      lds_barrier();   // both halves written; the partner's was read before the next tile's barrier
      const float* other = &s_xch[w_u ^ 2][0];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 p = *reinterpret_cast<const float4*>(other + (g * 64 + lane) * 4);
        sv[4 * g] += p.x;
        sv[4 * g + 1] += p.y;
        sv[4 * g + 2] += p.z;
        sv[4 * g + 3] += p.w;
      }
      return sv;
    } else {
      return s_tile_k(u, spread, std::integral_constant<int, 0>{}, [] {});
    }
  };

  // ---- raw scores of tile u: slots past the token list (partial last tile) masked
  auto mask_tile = [&](int u, f32x16& sv) __attribute__((always_inline)) {
    const int nvalid = ntok - u * BN;
    if (nvalid < BN) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int tk = row_tok((i >> 2) * 8 + kg * 4 + (i & 3));
        sv[i] = tk < nvalid ? sv[i] : -INFINITY;
      }
    }
  };

  // ---- online softmax of tile u for head hq (lane holds 16 raw scores; the scale is
  // positive, see cpos): P (io dtype) to pt[u & 1], the O rescale factor to
  // s_alpha[u & 1]. Branch-free, so the scheduler can place it among the PV MFMAs it
  // is issued with.
  auto softmax_tile = [&](int u, const f32x16& sv) __attribute__((always_inline)) {
    float mx = sv[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) mx = fmaxf(mx, sv[i]);
    // every tile holds at least one valid token: mx is finite; max(c s) = c max(s), c > 0
    mx = max_half_swap(mx) * cpos;
    m_true = fmaxf(m_true, mx);
    // lazy rescaling: the reference maximum moves only when the tile max exceeds it
    // by more than TAU; alpha is exactly 1 otherwise, and 1 on the first tile (O
    // and l are still zero)
    const float m_new = mx > m_used + lazy_tau<IO>() ? mx : m_used;
    const float alpha = m_used == -INFINITY ? 1.f : __builtin_amdgcn_exp2f((m_used - m_new) * LOG2E);
    m_used = m_new;
    const float mb = m_used * LOG2E;
    float psum = 0.f;
    uint16_t* prow = pt[u & 1] + hq * PP + kg * 4;
    const bool writer = !KSPLIT || kh == 0;   // one wave of a pair writes P and alpha
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      float p[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        p[j] = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[g * 4 + j], cl2, -mb));
        psum += p[j];
      }
      if (writer) *reinterpret_cast<uint2*>(prow + g * 8) = make_uint2(pack2<IO>(p[0], p[1]), pack2<IO>(p[2], p[3]));
    }
    l_part = l_part * alpha + psum;
    if (writer) s_alpha[u & 1][hq] = alpha;   // both lane halves hold the same head and value
  };

  // ---- O^T[this wave's D/4 columns, NH heads] += V^T P^T for tile u. Every operand (P
  // fragments of pt[u & 1] and transposed V reads for both 16-token steps) is
  // requested first; `between()` runs after the requests and before the MFMAs.
  auto pv_tile = [&](int u, auto&& between) __attribute__((always_inline)) {
    const uint8_t* nope = nope_buf[u % NBUF];
    const uint16_t* ptu = pt[u & 1];
    uint4 pa[KQ][MT], vb[KQ][C::NT];
#pragma unroll
    for (int kq = 0; kq < KQ; ++kq) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        pa[kq][mt] = *reinterpret_cast<const uint4*>(ptu + (mt * 32 + (lane & 31)) * PP + kq * 16 + kg * 8);
#pragma unroll
      for (int nt = 0; nt < C::NT; ++nt) {
        const int col = wave * C::DW + nt * 32 + (g16 & 1) * 16 + 4 * (c16 & 3);
        const int tok0 = kq * 16 + (g16 >> 1) * 8 + (c16 >> 2);
        const uint2 lo = ds_read_tr(nope + nope_off<D>(tok0) + col * 2);
        const uint2 hi = ds_read_tr(nope + nope_off<D>(tok0 + 4) + col * 2);
        vb[kq][nt] = make_uint4(lo.x, lo.y, hi.x, hi.y);
      }
    }
    between();
#pragma unroll
    for (int kq = 0; kq < KQ; ++kq)
#pragma unroll
      for (int nt = 0; nt < C::NT; ++nt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) o[mt][nt] = Mfma<IO>::m32(vb[kq][nt], pa[kq][mt], o[mt][nt]);
  };

  // ---- software pipeline over tiles. Iteration t: (barrier) rescale O for tile t,
  // S^T of tile t+1 with the loads of tile t+2 spread over it, then the PV MFMAs of
  // tile t with the softmax of tile t+1 placed between their operand reads and
  // the MFMAs, so the VALU softmax runs while the matrix core works. Buffers:
  // tile t (PV) and t+1 (S^T) are read, t+2 is loaded into the third; P and the
  // rescale factors are double-buffered by tile parity.
  if constexpr (TEACH) {
    // lane: token lane % 32 of the tile, heads 32 hb + m32_row(i, lane) of this wave's block
    const int hb = KSPLIT ? wave & 1 : wave;
    float tm[16], ti[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      tm[i] = t_mx[hb * 32 + m32_row(i, lane)];
      ti[i] = t_il[hb * 32 + m32_row(i, lane)];
    }
    const float sl2 = a.scale * LOG2E, inv_n1 = 1.f / n1;
    // this wave's head-block sum for every token of tile u, to t_tp[u & 1][wave]
    auto teach_write = [&](int u, const f32x16& sv) __attribute__((always_inline)) {
      float e = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) e += __builtin_amdgcn_exp2f(__builtin_fmaf(sv[i], sl2, -tm[i])) * ti[i];
      e = add_half_swap(e);   // lane l ^ 32 holds the block's other 16 heads of the token
      const int tok = lane & 31;
      if (lane < 32 && (!KSPLIT || kh == 0)) t_tp[((u & 1) * NWV + wave) * BN + tok] = u * BN + tok < ntok ? e : 0.f;
    };
    // the sums of tile u over the head blocks (written before the last barrier) to t_p
    auto teach_store = [&](int u) __attribute__((always_inline)) {
      const int tok = threadIdx.x;
      if (tok < BN && u * BN + tok < ntok) {
        float sum = 0.f;
#pragma unroll
        for (int w = 0; w < NWV; ++w)
          if (!KSPLIT || (w >> 1) == 0) sum += t_tp[((u & 1) * NWV + w) * BN + tok];
        a.t_p[(int64_t)r * a.t_ld + t_beg + u * BN + tok] = sum * inv_n1;
      }
    };
    wait_vmcnt<C::GPW - 1>();   // this wave's part of tile 0 landed; tile 1 may be in flight
    lds_barrier();
    teach_write(0, s_tile(0, [&](int) {}));
    for (int t = 0; t + 1 < ntiles; ++t) {
      if (t == 0) wait_vmcnt<0>(); else wait_vmcnt<1>();
      lds_barrier();   // tile t+1 resident and tile t's sums visible; tile t's buffer free
      teach_store(t);
      const TileIdx ix = tile_idx(t + 2);
      uint8_t* gnope = nope_buf[(t + 2) % NBUF];
      uint8_t* grope = rope_buf[(t + 2) % NBUF];
      teach_write(t + 1, s_tile(t + 1, [&](int ks) {
#pragma unroll
        for (int j = 0; j < C::GPW; ++j)
          if (j * KSH / C::GPW == ks) {
            if (j < C::GPW - 1) gather_part<D>(j, kb, krb, ws.zero, krows, ix, gnope, grope, wave_u, lane);
            else ids_dma(t + 4);
          }
      }));
      __builtin_amdgcn_sched_barrier(0);
    }
    wait_vmcnt<0>();   // the ring's last (unused) gathers land before the LDS is released
    lds_barrier();
    teach_store(ntiles - 1);
    return;
  }
  if constexpr (OWN) {
    // Lane's transposed-read base inside a nope buffer: tokens (g16/2)*8 + c16/4 (and +4,
    // the operand's upper half), columns (g16%2)*16 + 4(c16%4) of a 32-column tile -- the
    // pattern whose reads land on distinct banks. Token bit 2 is clear there, so
    // nope_off(t + 4) = nope_off(t) + 4 ROW + 16 and the 16-token steps add 16 ROW.
    const int vlane = nope_off<D>((g16 >> 1) * 8 + (c16 >> 2)) + ((g16 & 1) * 16 + 4 * (c16 & 3)) * 2;
    constexpr int NPV = 2 * ON;   // PV MFMAs per tile: two 16-token steps x ON column tiles
    constexpr int VR = 8;         // V^T operands in flight (8 MFMAs ahead: ~250 cycles)
    static_assert(NPV >= VR, "V^T operand ring");
    // the lane's LDS address in buffer `nope`, laundered so that each read's constant
    // offset goes into the instruction (the compiler would otherwise keep one
    // precomputed address per read in a VGPR)
    auto v_base = [&](const uint8_t* nope) __attribute__((always_inline)) -> uint32_t {
      uint32_t b = lds_addr(nope) + vlane;
      asm volatile("" : "+v"(b));
      return b;
    };
    auto v_frag = [&](uint32_t b, int m) __attribute__((always_inline)) -> uint4 {
      const uint32_t p = b + (m / ON) * 16 * C::ROW + (m % ON) * 64;
      const uint2 lo = ds_read_tr_at(p);
      const uint2 hi = ds_read_tr_at(p + 4 * C::ROW + 16);
      return make_uint4(lo.x, lo.y, hi.x, hi.y);
    };
    uint4 pb[2];         // P^T of the tile whose PV runs: B operands of its two 16-token steps
    uint4 pn[2];         // the same for the next tile (the softmax's output)
    float alpha = 1.f;   // O rescale factor of the next tile (the lane's head)
    float sm_mx = 0.f, sm_mb = 0.f, sm_sum = 0.f;
    uint32_t sm_d[4][2];
    constexpr int NST = 14;   // softmax stages, spread over the previous tile's PV MFMAs
    // Stage st of the online softmax of raw scores sv (lane: head hq, tokens 16 kq +
    // 8(lane/32) + j at sv[8 kq + j], see row_tok), each a few VALU ops: 0-3 the max over
    // four scores each, 4 the tile max and exponent reference, 5-12 two exponentials
    // each, 13 the row sum and the B operands of the two 16-token steps.
    auto smx = [&](int st, const f32x16& sv) __attribute__((always_inline)) {
      if (st < 4) {
        const int b = 4 * st;
        sm_mx = st == 0 ? fmaxf(fmaxf(sv[b], sv[b + 1]), fmaxf(sv[b + 2], sv[b + 3]))
                        : fmaxf(fmaxf(fmaxf(sm_mx, sv[b]), sv[b + 1]), fmaxf(sv[b + 2], sv[b + 3]));
      } else if (st == 4) {
        // every tile holds at least one valid token: the max is finite; max(c s) = c max(s), c > 0
        const float mx = max_half_swap(sm_mx) * cpos;
        m_true = fmaxf(m_true, mx);
        const float m_new = mx > m_used + lazy_tau<IO>() ? mx : m_used;   // lazy rescaling
        alpha = m_used == -INFINITY ? 1.f : __builtin_amdgcn_exp2f((m_used - m_new) * LOG2E);
        m_used = m_new;
        sm_mb = m_used * LOG2E;
        sm_sum = 0.f;
      } else if (st < NST - 1) {
        const int i = 2 * (st - 5);
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[i], cl2, -sm_mb));
        const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[i + 1], cl2, -sm_mb));
        sm_sum += p0;
        sm_sum += p1;
        sm_d[i >> 2][(i >> 1) & 1] = pack2<IO>(p0, p1);
      } else {
        l_part = l_part * alpha + sm_sum;
        pn[0] = make_uint4(sm_d[0][0], sm_d[0][1], sm_d[1][0], sm_d[1][1]);
        pn[1] = make_uint4(sm_d[2][0], sm_d[2][1], sm_d[3][0], sm_d[3][1]);
      }
    };
    // O *= alpha when the lane's head moved its exponent reference (rare: lazy rescaling)
    auto rescale = [&]() __attribute__((always_inline)) {
      if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {
#pragma unroll
        for (int nt = 0; nt < ON; ++nt)
#pragma unroll
          for (int i = 0; i < 16; ++i) o[0][nt][i] = agpr_scale(o[0][nt][i], alpha);
      }
    };
    // PV MFMAs [m0, m1) of a tile. The V^T operands run VR MFMAs ahead in one ring across
    // tiles: past the tile's last MFMA the reads continue with the next tile's first
    // operands (at LDS address `vnext`, resident since the barrier that preceded them).
    // `between(m)` runs after the m-th MFMA.
    constexpr int NPRE = 6;   // PV MFMAs issued before the next S^T chain (cover its operand latency)
    uint4 vb[VR];
    auto pv_run = [&](int m0, int m1, uint32_t vbase, uint32_t vnext, bool next, auto&& between)
        __attribute__((always_inline)) {
#pragma unroll
      for (int m = m0; m < m1; ++m) {
        o[0][m % ON] = Mfma<IO>::m32(vb[m % VR], pb[m / ON], o[0][m % ON]);
        if (m + VR < NPV) vb[m % VR] = v_frag(vbase, m + VR);
        else if (next) vb[m % VR] = v_frag(vnext, m + VR - NPV);
        between(m);
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    wait_vmcnt<C::GPW - 1>();   // this wave's part of tile 0 landed; tile 1 may be in flight
    lds_barrier();              // tile 0 visible
    {
      f32x16 s0 = s_tile(0, [&](int) {});
      mask_tile(0, s0);
#pragma unroll
      for (int st = 0; st < NST; ++st) smx(st, s0);
      const uint32_t vb0 = v_base(nope_buf[0]);
#pragma unroll
      for (int m = 0; m < VR; ++m) vb[m] = v_frag(vb0, m);
    }
    // Iteration t: O rescaled for tile t; after the barrier the first NPRE PV MFMAs of tile
    // t, the S^T chain of tile t+1 (carrying the gathers of tile t+2), then the other PV
    // MFMAs of tile t with the softmax of tile t+1 staged among them; the ring ends with
    // the first V^T operands of tile t+1.
    uint32_t zero_rows = 0;   // this wave's rows of tile t+1 to zero (ids out of range)
    for (int t = 0; t + 1 < ntiles; ++t) {
      pb[0] = pn[0];
      pb[1] = pn[1];
      rescale();   // tile t's factor (its softmax ran in the previous iteration)
      if (t == 0) wait_vmcnt<0>(); else wait_vmcnt<1>();   // this wave's gathers of tile t+1
      if (zero_rows) {   // rare: such rows read as zeros, as the zero row gives
        wait_vmcnt<0>();
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (((zero_rows >> j) & 1u) && lane < C::LANES_ROW)
            *reinterpret_cast<uint4*>(nope_buf[(t + 1) % NBUF] + nope_off<D>(wave_u * 8 + j) + lane * 16) =
                make_uint4(0, 0, 0, 0);
      }
      lds_barrier();   // tile t+1 resident; every wave's PV reads of tile t-1 done, so its buffer is free
      const TileIdx ix = tile_idx(t + 2, true);
      zero_rows = ix.zero_rows;
      uint8_t* gnope = nope_buf[(t + 2) % NBUF];
      uint8_t* grope = rope_buf[(t + 2) % NBUF];
      const uint32_t vbase = v_base(nope_buf[t % NBUF]);
      const uint32_t vnext = v_base(nope_buf[(t + 1) % NBUF]);
      f32x16 s1 = s_tile_k(
          t + 1,
          [&](int ks) {
#pragma unroll
            for (int j = 0; j < C::GPW; ++j)
              if (j * KSH / C::GPW == ks) {
                if (j < C::GPW - 1) gather_part<D, true>(j, kb, krb, ws.zero, krows, ix, gnope, grope, wave_u, lane);
                else ids_dma(t + 4);   // slot (t+4)%4 held the ids of tile t, read two iterations ago
              }
          },
          std::integral_constant<int, 0>{}, [&] { pv_run(0, NPRE, vbase, vnext, true, [](int) {}); });
      mask_tile(t + 1, s1);
      pv_run(NPRE, NPV, vbase, vnext, true, [&](int m) {
#pragma unroll
        for (int st = 0; st < NST; ++st)
          if (st * (NPV - NPRE) / NST == m - NPRE) smx(st, s1);
      });
      __builtin_amdgcn_sched_barrier(0);
    }
    pb[0] = pn[0];
    pb[1] = pn[1];
    rescale();
    pv_run(0, NPV, v_base(nope_buf[(ntiles - 1) % NBUF]), 0u, false, [](int) {});
    wait_vmcnt<0>();   // the ring's last (unused) gathers must land before the LDS is released
  } else {
  wait_vmcnt<C::GPW - 1>();   // this wave's part of tile 0 landed; tile 1 may be in flight
  lds_barrier();   // tile 0 visible
  {
    f32x16 s0 = s_tile(0, [&](int) {});
    mask_tile(0, s0);
    softmax_tile(0, s0);
  }
  // barrier at the top of iteration t, then rescale O by alpha(t) when any head's
  // factor differs from 1 (rare: lazy rescaling)
  auto tile_top = [&](int t) __attribute__((always_inline)) {
    // this wave's gathers of tile t+1 landed (the ids copy after them may be in
    // flight; at t = 0 nothing follows tile 1's gathers)
    if (t == 0)
      wait_vmcnt<0>();
    else
      wait_vmcnt<1>();
    lds_barrier();     // P and alpha of tile t visible; tile t+1 resident; PV of tile t-1 done everywhere
    const float a0 = s_alpha[t & 1][lane], a1 = NH > 64 ? s_alpha[t & 1][(lane + 64) % NH] : 1.f;
    if (__builtin_amdgcn_ballot_w64(a0 != 1.f || a1 != 1.f)) {
      // O^T layout: every element a lane holds in M tile mt belongs to head mt*32 + lane%32
#pragma unroll
      for (int mt = 0; mt < OM; ++mt) {
        const float al = s_alpha[t & 1][mt * 32 + (lane & 31)];
#pragma unroll
        for (int nt = 0; nt < ON; ++nt)
#pragma unroll
          for (int i = 0; i < 16; ++i) o[mt][nt][i] = agpr_scale(o[mt][nt][i], al);
      }
    }
  };
  // The last tile is peeled off the loop so the PV code is never duplicated
  // across the two arms of a branch (the merge would copy all of O).
  for (int t = 0; t + 1 < ntiles; ++t) {
    tile_top(t);
    const TileIdx ix = tile_idx(t + 2);
    uint8_t* gnope = nope_buf[(t + 2) % NBUF];   // held tile t-1, whose PV finished before the barrier
    uint8_t* grope = rope_buf[(t + 2) % NBUF];
    f32x16 s1 = s_tile(t + 1, [&](int ks) {
#pragma unroll
      for (int j = 0; j < C::GPW; ++j)
        if (j * KSH / C::GPW == ks) {
          if (j < C::GPW - 1) gather_part<D>(j, kb, krb, ws.zero, krows, ix, gnope, grope, wave_u, lane);
          else ids_dma(t + 4);   // slot (t+4)%4 held the ids of tile t, read two iterations ago
        }
    });
    mask_tile(t + 1, s1);
    pv_tile(t, [&]() { softmax_tile(t + 1, s1); });
    __builtin_amdgcn_sched_barrier(0);
  }
  tile_top(ntiles - 1);
  pv_tile(ntiles - 1, [&]() {});
  wait_vmcnt<0>();   // the ring's last (unused) gathers must land before the LDS is released
  }

  // ---- epilogue
  const float l_tot = l_part + __shfl_xor(l_part, 32);
  const bool owner = lane < 32 && kh == 0;   // one lane per head (a pair holds equal values)
  if (!OWN && owner) s_l[hq] = 1.f / l_tot;   // l > 0: a row or split holds at least one token
  if (direct) {
    if (owner && hq < n1 && a.sm_max) {
      a.sm_max[(int64_t)r * n1 + hq] = m_true;
      a.sm_sum[(int64_t)r * n1 + hq] = l_tot * exp2f((m_used - m_true) * LOG2E);
    }
  } else if (owner && hq < n1) {
    float* ps = ws.part_s + (((int64_t)r * splits + sp) * n1 + hq) * 3;
    ps[0] = m_used;
    ps[1] = m_true;
    ps[2] = l_tot;
  }
  // s_l (written only here) visible to every wave; an LDS-only barrier, so the
  // statistics stores above are not waited for (OWN: every lane holds its own head's l)
  if constexpr (!OWN) lds_barrier();
  // O^T layout: in accumulator (mt, nt) lane l holds head h = mt*32 + l%32 (OWN: the
  // wave's block) and, at index 4g + j, column c0 + nt*32 + 8g + 4(l/32) + j (g, j < 4;
  // c0 = wave*DW, or 0 for OWN). After scaling and packing, two lane-half swaps leave
  // lanes l < 32 with columns [0,8) and [16,24) of the 32-column group and lanes l >= 32
  // with [8,16) and [24,32): two 16-byte stores per accumulator instead of sixteen 2-byte ones.
#pragma unroll
  for (int mt = 0; mt < OM; ++mt) {
    const int h = (OWN ? wave : mt) * 32 + (lane & 31);
    const float inv = OWN ? 1.f / l_tot : s_l[h];
    // one split: the output row; several: this split's normalised partial
    uint16_t* orow = (direct ? out + ((int64_t)r * n1 + min(h, n1 - 1)) * D
                             : ws.part_o + (((int64_t)r * splits + sp) * n1 + min(h, n1 - 1)) * D) +
                     (OWN ? 0 : wave * C::DW) + (lane >> 5) * 8;
#pragma unroll
    for (int nt = 0; nt < ON; ++nt) {
      uint32_t d[4][2];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        d[g][0] = pack2<IO>(o[mt][nt][4 * g] * inv, o[mt][nt][4 * g + 1] * inv);
        d[g][1] = pack2<IO>(o[mt][nt][4 * g + 2] * inv, o[mt][nt][4 * g + 3] * inv);
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        swap_halves(d[0][j], d[1][j]);
        swap_halves(d[2][j], d[3][j]);
      }
      if (h < n1) {
        stg16(orow + nt * 32, make_uint4(d[0][0], d[0][1], d[1][0], d[1][1]));
        stg16(orow + nt * 32 + 16, make_uint4(d[2][0], d[2][1], d[3][0], d[3][1]));
      }
    }
  }
}

// ---------------------------------------------------------------- kernel 2, 64-head form (D = 512)
// One work-group of 8 waves (two per SIMD) per (query row, 64 heads, KV split), launched
// for N1 <= 64 (the reference's perf_sfa shape). O^T and Q^T of 64 heads take half the
// registers of the 128-head form, so two waves share each SIMD.
//  * S^T[32 tokens, 32 heads] of head block hb = w % 2 is split over the contraction:
//    wave w runs k-steps [9 q, 9 q + 9), q = w / 2 (Q^T fragments of those k-steps, rope
//    included, in VGPRs). The four partial sums meet in LDS; wave (hb, q) adds the
//    partials of token group q (tokens 8 q .. 8 q + 7: one 4-element group of the
//    32x32 accumulator) and runs the softmax of those tokens.
//  * Lazy rescaling across the four waves of a head block: P is computed against the
//    shared exponent reference m_used, and a wave whose group holds a score above
//    m_used + TAU raises a work-group flag. Every wave reads the flag after the next
//    barrier; on that (rare) path the group maxima are read back, m_used moves to the
//    tile maximum, P is recomputed from the scores kept in registers and O is rescaled,
//    behind one more barrier. The first tile always takes it (m_used starts at -inf).
//    The true maximum and the row sum are per wave and combined at the end.
//  * Each wave owns 64 columns of O^T[512, 64 heads] and accumulates O^T += V^T P^T as
//    the 128-head form does; the PV MFMAs of the previous tile are split around the
//    exchange barrier so the matrix core has work while the partial sums travel.
//  * Gathers: wave w copies the nope rows of tokens 4w .. 4w + 3, waves 0-3 the rope of
//    tokens 8w .. 8w + 7, every wave its 4 ids of the tile four ahead (the last load of
//    an iteration, so one vmcnt wait retires a tile in every wave).
//  * Rows of more than 64 heads would run as two halves launched 8 work-groups apart
//    (round-robin dispatch over the 8 XCDs puts them on one XCD, whose L2 then serves
//    both halves' gathers); the launcher keeps such rows on the 128-head form.
namespace w8 {
constexpr int NW = 8;          // waves
constexpr int HH = 64;         // heads per work-group
constexpr int DD = 512;
constexpr int KS = (DD + DR) / 16;   // S^T k-steps (36)
constexpr int KSN = DD / 16;         // of which nope (32)
constexpr int KQ = KS / 4;           // k-steps per wave (9)
constexpr int PPH = BN + 8;          // P tile pitch (elements)
}  // namespace w8

template <int IO>
__global__ __launch_bounds__(w8::NW * 64) void sfa_attn8_kernel(SfaArgs a, int splits, Ws ws) {
  using C = Cfg<w8::DD>;
  constexpr int D = w8::DD;
  __shared__ __attribute__((aligned(16))) uint8_t nope_buf[NBUF][C::NOPE];
  __shared__ __attribute__((aligned(16))) uint8_t rope_buf[NBUF][C::ROPE];
  __shared__ __attribute__((aligned(16))) uint16_t pt[2][w8::HH * w8::PPH];   // P [head][token], by tile parity
  __shared__ __attribute__((aligned(16))) float4 xch[2][4][3][64];   // S^T partials [hb][token group][source][lane]
  __shared__ __attribute__((aligned(16))) int32_t s_ids[4][BN];      // token-id ring (tiles t+2 .. t+4)
  __shared__ __attribute__((aligned(16))) float s_mx[2][w8::HH][4];   // group maxima [parity][head][group]
  __shared__ float s_alpha[w8::HH];   // O rescale factors (rare path)
  __shared__ int s_flag[2];           // a group exceeded m_used + TAU, by tile parity

  // (row, head half, split) of this work-group; halves of one (row, split) 8 apart
  const int nh = a.n1 > w8::HH ? 2 : 1;
  const int nq = a.total_rows * splits;
  const int x = blockIdx.x;
  const int q = nh == 2 ? (x >> 4) * 8 + (x & 7) : x;
  const int hh = nh == 2 ? (x >> 3) & 1 : 0;
  if (q >= nq) return;
  const int sp = q / a.total_rows;
  const int r = a.total_rows - 1 - (q - sp * a.total_rows);   // long (late causal) rows first

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave_u = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hb = wave_u & 1, kq = wave_u >> 1;
  const int n1 = a.n1;
  const int h0 = hh * w8::HH;
  const int hl = hb * 32 + (lane & 31);   // local head of this lane's S^T column
  const int hs = h0 + hl;
  const int ntok_all = ws.counts[r];
  // Q^T fragments of k-steps 9 kq + j (nope, then rope), clamped heads zeroed below
  uint4 qf[w8::KQ];
  {
    const int hc = hs < n1 ? hs : n1 - 1;
    const uint16_t* qn = reinterpret_cast<const uint16_t*>(a.q) + ((int64_t)r * n1 + hc) * D + (lane >> 5) * 8;
    const uint16_t* qrr = reinterpret_cast<const uint16_t*>(a.qr) + ((int64_t)r * n1 + hc) * DR + (lane >> 5) * 8;
#pragma unroll
    for (int j = 0; j < w8::KQ; ++j) {
      const int ks = kq * w8::KQ + j;
      qf[j] = ldg16(ks < w8::KSN ? qn + ks * 16 : qrr + (ks - w8::KSN) * 16);
    }
    asm volatile("" ::: "memory");   // the loads stay ahead of the token-count branch
  }
  const int per = ((ntok_all + splits - 1) / splits + BN - 1) / BN * BN;
  const int t_beg = sp * per;
  const int t_end = (t_beg + per < ntok_all ? t_beg + per : ntok_all);
  const int ntok = t_end > t_beg ? t_end - t_beg : 0;
  const int32_t* toks = ws.tokens + (int64_t)r * ws.tstride + t_beg;
  uint16_t* out = reinterpret_cast<uint16_t*>(a.out);
  if (ntok == 0) {
    wait_vmcnt<0>();
    if (ntok_all == 0 && sp == 0) {   // skipped row: zeros (out, stats) for this half's heads
      const int hn = n1 - h0 < w8::HH ? n1 - h0 : w8::HH;
      for (int i = tid; i < hn * D / 8; i += w8::NW * 64)
        stg16(out + ((int64_t)r * n1 + h0) * D + i * 8, make_uint4(0, 0, 0, 0));
      if (a.sm_max)
        for (int h = tid; h < hn; h += w8::NW * 64) {
          a.sm_max[(int64_t)r * n1 + h0 + h] = 0.f;
          a.sm_sum[(int64_t)r * n1 + h0 + h] = 0.f;
        }
    }
    return;
  }
  const int nact = (ntok_all + per - 1) / per;
  const bool direct = nact == 1;
  const uint16_t* kb = reinterpret_cast<const uint16_t*>(a.k);
  const uint16_t* krb = reinterpret_cast<const uint16_t*>(a.kr);
  const int krows = a.key_rows < INT_MAX ? (int)a.key_rows : INT_MAX;
  const int ntiles = (ntok + BN - 1) / BN;
  const int tr = lane & 31, kg = lane >> 5;
  const int g16 = lane >> 4, c16 = lane & 15;

  auto clamp_tile = [&](int t) { return t < ntiles ? t : ntiles - 1; };
  // this wave's 4 ids of tile t into ring slot t % 4 (tiles past the end re-read the last)
  auto ids_dma = [&](int t) {
    if (lane == 0) lds_dma16_sbase_untracked(toks + clamp_tile(t) * BN + wave_u * 4, 0u, &s_ids[t & 3][wave_u * 4]);
  };
  // ids of tile t: x = token lane % 32 (the nope rows, by readlane), y = the rope token
  // 8 (w % 4) + lane % 8; slots past the token list take the tile's first token
  auto tile_ids = [&](int t) {
    const int nvalid = ntok - clamp_tile(t) * BN < BN ? ntok - clamp_tile(t) * BN : BN;
    const int k1 = lane & 31, k2 = 8 * (wave_u & 3) + (lane & 7);
    const int first = s_ids[t & 3][0];
    const int v1 = s_ids[t & 3][k1], v2 = s_ids[t & 3][k2];
    return make_int2(k1 < nvalid ? v1 : first, k2 < nvalid ? v2 : first);
  };
  // gather part j of a tile: j < 4 the nope row of token 4w + j (all 64 lanes, one row),
  // j = 4 the rope chunks of tokens 8w .. 8w + 7 (waves 0-3). Rows outside the key
  // tensors read the zero row.
  auto gather_part8 = [&](int j, int2 idv, uint8_t* nope, uint8_t* rope) __attribute__((always_inline)) {
    if (j < 4) {
      const int phys = __builtin_amdgcn_readlane(idv.x, wave_u * 4 + j);
      const uint16_t* src = (uint32_t)phys < (uint32_t)krows ? kb + (int64_t)phys * D : ws.zero;
      lds_dma16_sbase_untracked(src, lane * 16, nope + nope_off<D>(wave_u * 4 + j));
    } else if (wave_u < 4) {
      const uint16_t* src = (uint32_t)idv.y < (uint32_t)krows ? krb + (int64_t)idv.y * DR : ws.zero + 512;
      lds_dma16_untracked(src + (lane >> 3) * 8, rope + wave_u * 1024);
    }
  };

  // ---- prologue: ids of tiles 0..3, Q landed, flags cleared, then the first two gathers
#pragma unroll
  for (int t = 0; t < 4; ++t) ids_dma(t);
  wait_vmcnt<0>();
  if (hs >= n1)
#pragma unroll
    for (int j = 0; j < w8::KQ; ++j) qf[j] = make_uint4(0, 0, 0, 0);
  if (tid < 2) s_flag[tid] = 0;
  lds_barrier();
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int2 idv = tile_ids(u);
#pragma unroll
    for (int j = 0; j < 5; ++j) gather_part8(j, idv, nope_buf[u], rope_buf[u]);
  }

  float m_used = -INFINITY, m_true = -INFINITY, l_part = 0.f, l_prev = 0.f;
  float s_keep[4] = {0.f, 0.f, 0.f, 0.f};
  f32x16 o[2][2];   // O^T [head block mt][column block nt]
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[mt][nt][i] = 0.f;

  // ---- partial S^T[32 tokens, 32 heads of hb] of tile u over this wave's 9 k-steps;
  // spread(j) issues the loads scheduled after step j
  auto s_part = [&](int u, auto&& spread) __attribute__((always_inline)) -> f32x16 {
    const uint8_t* nope = nope_buf[u % NBUF];
    const uint8_t* rope = rope_buf[u % NBUF];
    const uint8_t* arow = nope + nope_off<D>(tr) + kg * 16;
    const int k0 = kq * w8::KQ;
    auto a_frag = [&](int ks) -> uint4 {
      return ks < w8::KSN ? *reinterpret_cast<const uint4*>(arow + ks * 32)
                          : *reinterpret_cast<const uint4*>(rope + rope_off(tr, (ks - w8::KSN) * 2 + kg));
    };
    f32x16 sacc = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    uint4 af[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) af[j] = a_frag(k0 + j);
#pragma unroll
    for (int j = 0; j < w8::KQ; ++j) {
      sacc = Mfma<IO>::m32(af[j & 3], qf[j], sacc);
      if (j + 4 < w8::KQ) af[j & 3] = a_frag(k0 + j + 4);
      spread(j);
      __builtin_amdgcn_sched_barrier(0);
    }
    return sacc;
  };
  // the three token groups this wave does not own go to LDS
  auto xch_write = [&](const f32x16& sv) __attribute__((always_inline)) {
#pragma unroll
    for (int g = 0; g < 4; ++g)
      if (g != kq) xch[hb][g][kq < g ? kq : kq - 1][lane] = make_float4(sv[4 * g], sv[4 * g + 1], sv[4 * g + 2], sv[4 * g + 3]);
  };
  // this wave's group kq: its own partial plus the other three
  auto xch_sum = [&](const f32x16& sv) __attribute__((always_inline)) -> float4 {
    float4 s;
    s.x = kq == 0 ? sv[0] : kq == 1 ? sv[4] : kq == 2 ? sv[8] : sv[12];
    s.y = kq == 0 ? sv[1] : kq == 1 ? sv[5] : kq == 2 ? sv[9] : sv[13];
    s.z = kq == 0 ? sv[2] : kq == 1 ? sv[6] : kq == 2 ? sv[10] : sv[14];
    s.w = kq == 0 ? sv[3] : kq == 1 ? sv[7] : kq == 2 ? sv[11] : sv[15];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const float4 p = xch[hb][kq][j][lane];
      s.x += p.x;
      s.y += p.y;
      s.z += p.z;
      s.w += p.w;
    }
    return s;
  };
  // P of this wave's 4 tokens (lane) against m_used into pt[u & 1]; returns the sum
  auto write_p = [&](int u) __attribute__((always_inline)) -> float {
    const float mb = m_used * LOG2E;
    float p[4], psum = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s_keep[i], LOG2E, -mb));
      psum += p[i];
    }
    *reinterpret_cast<uint2*>(pt[u & 1] + hl * w8::PPH + 8 * kq + 4 * kg) =
        make_uint2(pack2<IO>(p[0], p[1]), pack2<IO>(p[2], p[3]));
    return psum;
  };
  // softmax of tile u for token group kq (tokens 8 kq + 4 (lane / 32) + i, head hl)
  auto softmax8 = [&](int u, float4 sg) __attribute__((always_inline)) {
    s_keep[0] = sg.x * a.scale;
    s_keep[1] = sg.y * a.scale;
    s_keep[2] = sg.z * a.scale;
    s_keep[3] = sg.w * a.scale;
    const int nvalid = ntok - u * BN;
    if (nvalid < BN)
#pragma unroll
      for (int i = 0; i < 4; ++i) s_keep[i] = 8 * kq + 4 * kg + i < nvalid ? s_keep[i] : -INFINITY;
    float mx = fmaxf(fmaxf(s_keep[0], s_keep[1]), fmaxf(s_keep[2], s_keep[3]));
    mx = max_half_swap(mx);
    if (lane < 32) s_mx[u & 1][hl][kq] = mx;
    m_true = fmaxf(m_true, mx);
    if (__builtin_amdgcn_ballot_w64(mx > m_used + lazy_tau<IO>()) && lane == 0) s_flag[u & 1] = 1;
    l_prev = l_part;
    l_part += write_p(u);
  };
  // the rare path for tile u (flag raised): m_used to the tile maximum where it moved,
  // P rewritten, O rescaled
  auto rare = [&](int u) __attribute__((always_inline)) {
    const float4 mq = *reinterpret_cast<const float4*>(&s_mx[u & 1][hl][0]);
    const float mt = fmaxf(fmaxf(mq.x, mq.y), fmaxf(mq.z, mq.w));
    const float m_new = mt > m_used + lazy_tau<IO>() ? mt : m_used;
    const float alpha = __builtin_amdgcn_exp2f((m_used - m_new) * LOG2E);   // 0 on the first tile
    m_used = m_new;
    l_part = l_prev * alpha + write_p(u);
    if (kq == 0 && lane < 32) s_alpha[hl] = alpha;
    lds_barrier();   // P rewritten, alpha written, the flag read by every wave
    if (tid == 0) s_flag[u & 1] = 0;
    const float a0 = s_alpha[lane & 31], a1 = s_alpha[32 + (lane & 31)];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        o[0][nt][i] *= a0;
        o[1][nt][i] *= a1;
      }
  };
  // PV operands of tile u, k-step ks (16 tokens): P^T fragments of both head blocks and
  // V^T fragments of this wave's two 32-column blocks
  auto pv_req = [&](int u, int ks, uint4 (&pa)[2], uint4 (&vb)[2]) __attribute__((always_inline)) {
    const uint8_t* nope = nope_buf[u % NBUF];
    const uint16_t* ptu = pt[u & 1];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
      pa[mt] = *reinterpret_cast<const uint4*>(ptu + (mt * 32 + (lane & 31)) * w8::PPH + ks * 16 + kg * 8);
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int col = wave_u * 64 + nt * 32 + (g16 & 1) * 16 + 4 * (c16 & 3);
      const int tok0 = ks * 16 + (g16 >> 1) * 8 + (c16 >> 2);
      const uint2 lo = ds_read_tr(nope + nope_off<D>(tok0) + col * 2);
      const uint2 hi = ds_read_tr(nope + nope_off<D>(tok0 + 4) + col * 2);
      vb[nt] = make_uint4(lo.x, lo.y, hi.x, hi.y);
    }
  };
  auto pv_mfma = [&](const uint4 (&pa)[2], const uint4 (&vb)[2]) __attribute__((always_inline)) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) o[mt][nt] = Mfma<IO>::m32(vb[nt], pa[mt], o[mt][nt]);
  };
  // barrier at the top of iteration t (tile t+1 resident, P(t) and its flag visible),
  // then the rare path of tile t when flagged
  auto tile_top = [&](int t) __attribute__((always_inline)) {
    if (t == 0)
      wait_vmcnt<0>();
    else
      wait_vmcnt<1>();
    lds_barrier();
    if (__builtin_amdgcn_readfirstlane(s_flag[t & 1])) rare(t);
  };

  // ---- tile 0: this wave's gathers of tile 0 landed (tile 1's may be in flight)
  if (wave_u < 4)
    wait_vmcnt<5>();
  else
    wait_vmcnt<4>();
  lds_barrier();
  {
    const f32x16 s0 = s_part(0, [&](int) {});
    xch_write(s0);
    lds_barrier();
    softmax8(0, xch_sum(s0));
  }
  // ---- iteration t: S^T of tile t+1 (gathers of tile t+2 spread over it), the first
  // half of PV(t), the partial exchange, then the softmax of tile t+1 beside the second
  // half of PV(t). Buffers: t (PV) and t+1 (S^T) read, t+2 loading; P by parity.
  for (int t = 0; t + 1 < ntiles; ++t) {
    tile_top(t);
    const int2 idv = tile_ids(t + 2);
    uint8_t* gnope = nope_buf[(t + 2) % NBUF];   // held tile t-1, whose PV finished before the barrier
    uint8_t* grope = rope_buf[(t + 2) % NBUF];
    const f32x16 s1 = s_part(t + 1, [&](int j) {
      if (j >= 1 && j <= 5) gather_part8(j - 1, idv, gnope, grope);
      if (j == 7) ids_dma(t + 4);   // slot (t+4)%4 held the ids of tile t, read two iterations ago
    });
    uint4 pa0[2], vb0[2], pa1[2], vb1[2];
    pv_req(t, 0, pa0, vb0);
    pv_req(t, 1, pa1, vb1);
    pv_mfma(pa0, vb0);
    xch_write(s1);
    lds_barrier();   // partials of tile t+1 visible
    softmax8(t + 1, xch_sum(s1));
    pv_mfma(pa1, vb1);
    __builtin_amdgcn_sched_barrier(0);
  }
  tile_top(ntiles - 1);
  {
    uint4 pa0[2], vb0[2], pa1[2], vb1[2];
    pv_req(ntiles - 1, 0, pa0, vb0);
    pv_req(ntiles - 1, 1, pa1, vb1);
    pv_mfma(pa0, vb0);
    pv_mfma(pa1, vb1);
  }
  wait_vmcnt<0>();   // the ring's last (unused) gathers land before the LDS is released

  // ---- epilogue: per head, the four group waves' sums and true maxima
  const float l_w = add_half_swap(l_part);   // lanes l and l ^ 32 hold other tokens of the head
  float2* red = reinterpret_cast<float2*>(&xch[0][0][0][0]);   // [head][group]
  lds_barrier();   // the last exchange reads are done
  if (lane < 32) red[hl * 4 + kq] = make_float2(l_w, m_true);
  lds_barrier();
  float inv[2];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    const int h = mt * 32 + (lane & 31);
    float lt = 0.f, mtr = -INFINITY;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float2 v = red[h * 4 + g];
      lt += v.x;
      mtr = fmaxf(mtr, v.y);
    }
    inv[mt] = 1.f / lt;   // l > 0: a row or split holds at least one token
    // statistics: wave (hb = mt, kq = 0) holds m_used of these heads
    if (kq == 0 && hb == mt && lane < 32 && h0 + h < n1) {
      const int64_t hr = (int64_t)r * n1 + h0 + h;
      if (direct) {
        if (a.sm_max) {
          a.sm_max[hr] = mtr;
          a.sm_sum[hr] = lt * exp2f((m_used - mtr) * LOG2E);
        }
      } else {
        float* ps = ws.part_s + (((int64_t)r * splits + sp) * n1 + h0 + h) * 3;
        ps[0] = m_used;
        ps[1] = mtr;
        ps[2] = lt;
      }
    }
  }
  // O^T layout: in accumulator (mt, nt) lane l holds head mt*32 + l%32 and, at index
  // 4g + j, column 64 w + 32 nt + 8g + 4(l/32) + j; packed, then two lane-half swaps
  // leave 16-byte runs (as in the 128-head form)
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    const int ha = h0 + mt * 32 + (lane & 31);
    const int hc = ha < n1 ? ha : n1 - 1;
    uint16_t* orow = (direct ? out + ((int64_t)r * n1 + hc) * D
                             : ws.part_o + (((int64_t)r * splits + sp) * n1 + hc) * D) +
                     wave_u * 64 + (lane >> 5) * 8;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      uint32_t d[4][2];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        d[g][0] = pack2<IO>(o[mt][nt][4 * g] * inv[mt], o[mt][nt][4 * g + 1] * inv[mt]);
        d[g][1] = pack2<IO>(o[mt][nt][4 * g + 2] * inv[mt], o[mt][nt][4 * g + 3] * inv[mt]);
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        swap_halves(d[0][j], d[1][j]);
        swap_halves(d[2][j], d[3][j]);
      }
      if (ha < n1) {
        stg16(orow + nt * 32, make_uint4(d[0][0], d[0][1], d[1][0], d[1][1]));
        stg16(orow + nt * 32 + 16, make_uint4(d[2][0], d[2][1], d[3][0], d[3][1]));
      }
    }
  }
}

template <int IO, int D>
hipError_t launch_attn_d(const SfaArgs& a, hipStream_t s, int cap, int splits, int fuse_tok, Ws ws) {
  // N1 <= 64: the 8-wave form (one work-group per row). Above 64 heads the 128-head form:
  // split into two 64-head work-groups a row pays two serial prologues and its tiles run
  // at about 1.5x the 128-head form's cycles (measured), so it stays one work-group.
  if (D == w8::DD && !fuse_tok && a.n1 <= w8::HH) {   // token lists built by the token-list launch
    const int64_t nq = (int64_t)a.total_rows * splits;
    const int64_t grid = a.n1 > w8::HH ? (nq + 7) / 8 * 16 : nq;
    hipLaunchKernelGGL(sfa_attn8_kernel<IO>, dim3((unsigned)grid), dim3(w8::NW * 64), 0, s, a, splits, ws);
  } else if (a.n1 <= 64)
    hipLaunchKernelGGL((sfa_attn_kernel<IO, D, 64, false>), dim3(a.total_rows, splits), dim3(NWV * 64), 0, s, a,
                       cap, splits, fuse_tok, ws);
  else if ((uint64_t)a.key_rows * D * 2 <= (1ull << 32))   // its gathers use 32-bit row offsets
    hipLaunchKernelGGL((sfa_attn_kernel<IO, D, 128, false, true>), dim3(a.total_rows, splits), dim3(NWV * 64), 0, s,
                       a, cap, splits, fuse_tok, ws);
  else
    hipLaunchKernelGGL((sfa_attn_kernel<IO, D, 128, false>), dim3(a.total_rows, splits), dim3(NWV * 64), 0, s, a,
                       cap, splits, fuse_tok, ws);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || splits == 1) return e;
  const int units = a.n1 * (D / 8);
  if (splits <= 4)
    hipLaunchKernelGGL((sfa_merge_kernel<IO, D, 4>), dim3(a.total_rows, (units + 255) / 256), dim3(256), 0,
                       s, a, splits, ws);
  else
    hipLaunchKernelGGL((sfa_merge_kernel<IO, D, 16>), dim3(a.total_rows, (units + 255) / 256), dim3(256), 0,
                       s, a, splits, ws);
  return hipGetLastError();
}

template <int IO, int D>
hipError_t launch_teach_d(const SfaArgs& a, hipStream_t s, int cap, Ws ws) {
  if (a.n1 <= 64)
    hipLaunchKernelGGL((sfa_attn_kernel<IO, D, 64, true>), dim3(a.total_rows, 1), dim3(NWV * 64), 0, s, a, cap, 1, 0,
                       ws);
  else
    hipLaunchKernelGGL((sfa_attn_kernel<IO, D, 128, true>), dim3(a.total_rows, 1), dim3(NWV * 64), 0, s, a, cap, 1,
                       0, ws);
  return hipGetLastError();
}

// The KL losses' slot list of row r = b * t_s1 + s1 as key rows of the BSND key tensor: the
// first n = min(topk, max(act_k - act_q + s1 + 1, 0)) slots (rows s1 >= act_q: none), slot i
// = sidx[r][i] clipped to [0, S2 - 1] (i itself without sidx), at key row b * S2 + id.
__global__ __launch_bounds__(TOK_TPB) void sfa_slot_list_kernel(SfaArgs a, Ws ws) {
  const int r = blockIdx.x;
  const int tid = threadIdx.x;
  if (r == 0)
    for (int i = tid; i < 512 + DR; i += TOK_TPB) ws.zero[i] = 0;
  const int b = r / a.t_s1, s1 = r - b * a.t_s1;
  const int aq = a.act_q[b], ak = a.act_k[b];
  int n = 0;
  if (s1 < aq) {
    n = ak - aq + s1 + 1;
    n = n < 0 ? 0 : (n < a.topk ? n : a.topk);
  }
  const int32_t* ids = a.sidx ? a.sidx + (int64_t)r * a.topk : nullptr;
  int32_t* out = ws.tokens + (int64_t)r * ws.tstride;
  for (int i = tid; i < n; i += TOK_TPB) {
    int id = ids ? ids[i] : i;
    id = id < 0 ? 0 : (id > a.s2 - 1 ? a.s2 - 1 : id);
    out[i] = b * a.s2 + id;
  }
  if (tid == 0) ws.counts[r] = n;
}

template <int IO>
hipError_t launch_attn(const SfaArgs& a, hipStream_t s, int cap, int splits, int fuse_tok, Ws ws) {
  switch (a.d) {
    case 128: return launch_attn_d<IO, 128>(a, s, cap, splits, fuse_tok, ws);
    case 256: return launch_attn_d<IO, 256>(a, s, cap, splits, fuse_tok, ws);
    case 512: return launch_attn_d<IO, 512>(a, s, cap, splits, fuse_tok, ws);
  }
  return hipErrorInvalidValue;
}

}  // namespace
}  // namespace dsa

// KV splits: unsplit for prefill-sized row counts; few rows (decode) are split so
// the grid covers the 256 CUs, keeping at least 4 tiles per split.
static int sfa_splits(int total_rows, int cap, int kv_splits) {
  if (kv_splits > 0) return kv_splits;
  if (total_rows >= 256) return 1;
  int s = (256 + total_rows - 1) / total_rows;
  const int max_s = cap / (4 * 32);
  if (s > max_s) s = max_s;
  if (s > 16) s = 16;
  return s < 1 ? 1 : s;
}

size_t sfa_workspace_zero_bytes() { return dsa::align256((size_t)(512 + dsa::DR) * 2); }   // the zero KV row

size_t sfa_workspace_bytes(int total_rows, int n1, int d, int topk, int sbs, int kv_splits) {
  const int cap = topk * sbs;
  size_t total = 0;
  dsa::ws_layout(nullptr, total_rows, cap, n1, d, sfa_splits(total_rows, cap, kv_splits), &total);
  return total;
}

size_t sfa_token_ws_bytes(int total_rows, int topk, int sbs) {
  size_t total = 0;
  dsa::ws_layout(nullptr, total_rows, topk * sbs, 1, 128, 1, &total);
  return total;
}

hipError_t launch_sfa_token_lists(const SfaArgs& a, void* ws_base, SfaTokenLists* tl, hipStream_t s) {
  const int cap = a.topk * a.sbs;
  dsa::Ws ws = dsa::ws_layout(ws_base, a.total_rows, cap, a.n1, a.d, 1, nullptr);
  tl->counts = ws.counts;
  tl->tokens = ws.tokens;
  tl->tstride = ws.tstride;
  if (a.total_rows <= 0) return hipSuccess;
  if (a.sbs == 1 && a.total_rows >= 256)
    hipLaunchKernelGGL(dsa::sfa_tokens1_kernel, dim3((a.total_rows + dsa::TOK1_ROWS - 1) / dsa::TOK1_ROWS),
                       dim3(64 * dsa::TOK1_ROWS), 0, s, a, cap, ws);
  else
    hipLaunchKernelGGL(dsa::sfa_tokens_kernel, dim3(a.total_rows), dim3(dsa::TOK_TPB), 0, s, a, cap, ws);
  return hipGetLastError();
}

// ---------------------------------------------------------------- no-allocation workspace
// dsa_sfa_fwd_noalloc runs the same launches on a file-scope device array instead of a
// caller-allocated workspace. Its name is only a host-side handle: host code uses the
// per-device address hipGetSymbolAddress returns, never the name itself.
namespace {
static __device__ __align__(256) uint8_t scratch[DSA_SFA_NOALLOC_SCRATCH_BYTES];

constexpr int SCRATCH_MAX_DEVICES = 64;
struct DeviceScratch {
  void* ptr = nullptr;   // this device's copy of `scratch`
  bool zeroed = false;   // its zero-row prefix cleared (by a synchronised, uncaptured launch)
};
std::mutex g_scratch_mu;
DeviceScratch g_scratch[SCRATCH_MAX_DEVICES];

__global__ void sfa_zero_prefix_kernel(uint4* p, int n16) {
  for (int i = threadIdx.x; i < n16; i += blockDim.x) p[i] = make_uint4(0, 0, 0, 0);
}
}  // namespace

hipError_t sfa_noalloc_workspace(hipStream_t s, void** ws) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= SCRATCH_MAX_DEVICES) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  DeviceScratch& d = g_scratch[dev];
  if (d.ptr == nullptr) {   // once per device, with that device current
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    d.ptr = p;
  }
  if (!d.zeroed) {
    // The zero KV row at the start of the workspace must read as zeros. The clear goes
    // on the caller's stream ahead of the call's own launches; outside stream capture it
    // is waited for once and never repeated, under capture it is part of every captured
    // call until an uncaptured one has run.
    const int n16 = (int)(sfa_workspace_zero_bytes() / 16);
    hipLaunchKernelGGL(sfa_zero_prefix_kernel, dim3(1), dim3(256), 0, s, reinterpret_cast<uint4*>(d.ptr), n16);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(s, &st);
    if (e != hipSuccess) return e;
    if (st == hipStreamCaptureStatusNone) {
      e = hipStreamSynchronize(s);
      if (e != hipSuccess) return e;
      d.zeroed = true;
    }
  }
  *ws = d.ptr;
  return hipSuccess;
}

hipError_t launch_sfa_teacher(const SfaArgs& a, hipStream_t s) {
  if (a.total_rows <= 0) return hipSuccess;
  const int cap = a.topk;
  dsa::Ws ws = dsa::ws_layout(a.ws, a.total_rows, cap, a.n1, a.d, 1, nullptr);
  hipLaunchKernelGGL(dsa::sfa_slot_list_kernel, dim3(a.total_rows), dim3(dsa::TOK_TPB), 0, s, a, ws);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const bool bf = a.io == dsa::IO_BF16;
  switch (a.d) {
    case 128: return bf ? dsa::launch_teach_d<dsa::IO_BF16, 128>(a, s, cap, ws) : dsa::launch_teach_d<dsa::IO_F16, 128>(a, s, cap, ws);
    case 256: return bf ? dsa::launch_teach_d<dsa::IO_BF16, 256>(a, s, cap, ws) : dsa::launch_teach_d<dsa::IO_F16, 256>(a, s, cap, ws);
    case 512: return bf ? dsa::launch_teach_d<dsa::IO_BF16, 512>(a, s, cap, ws) : dsa::launch_teach_d<dsa::IO_F16, 512>(a, s, cap, ws);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_sfa_fwd(const SfaArgs& a, hipStream_t s) {
  if (a.total_rows <= 0) return hipSuccess;
  const int cap = a.topk * a.sbs;
  const int splits = sfa_splits(a.total_rows, cap, a.kv_splits);
  dsa::Ws ws = dsa::ws_layout(a.ws, a.total_rows, cap, a.n1, a.d, splits, nullptr);
  // KV-split rows with sparse_block_size 1 (decode): each split lists its own
  // tokens inside the attention kernel, so no token-list launch precedes it.
  // Otherwise: one wave per row pays off once there are enough rows to fill the
  // GPU; a few rows are spread over a whole work-group each.
  const int fuse_tok = splits > 1 && a.sbs == 1;
  if (!fuse_tok) {
    if (a.sbs == 1 && a.total_rows >= 256)
      hipLaunchKernelGGL(dsa::sfa_tokens1_kernel, dim3((a.total_rows + dsa::TOK1_ROWS - 1) / dsa::TOK1_ROWS),
                         dim3(64 * dsa::TOK1_ROWS), 0, s, a, cap, ws);
    else
      hipLaunchKernelGGL(dsa::sfa_tokens_kernel, dim3(a.total_rows), dim3(dsa::TOK_TPB), 0, s, a, cap, ws);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return a.io == dsa::IO_BF16 ? dsa::launch_attn<dsa::IO_BF16>(a, s, cap, splits, fuse_tok, ws)
                              : dsa::launch_attn<dsa::IO_F16>(a, s, cap, splits, fuse_tok, ws);
}
