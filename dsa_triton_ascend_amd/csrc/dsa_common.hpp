// Shared device helpers for the gfx950 (CDNA4) DSA kernels.
//
// 16-bit floats are moved as raw uint16 bit patterns; the MFMA operands are
// 8-wide bf16 / fp16 vectors built from one 16-byte load. Conversions that the
// reference goldens define bit-exactly (fp32 -> bf16 round-to-nearest-even,
// lightning_indexer_numpy.py:20-24) are restated here on the bit pattern.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/dsa_mi355x.h"

namespace dsa {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

enum IoType { IO_F16 = DSA_DTYPE_F16, IO_BF16 = DSA_DTYPE_BF16 };

// ------------------------------------------------------------------ conversions
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(((uint32_t)h) << 16);
}
// Round-to-nearest-even fp32 -> bf16 (gfx950 v_cvt_pk_bf16_f32). For finite
// inputs this equals the golden's bit rule (add 0x7FFF plus the lsb of the kept
// half, then truncate), lightning_indexer_numpy.py:20-24.
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}
__device__ __forceinline__ uint16_t f32_to_f16_rne(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);  // v_cvt_f16_f32, RNE
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two fp32 values -> two RNE-rounded 16-bit values packed in one dword (lo = a).
template <int IO> __device__ __forceinline__ uint32_t pack2(float a, float b) {
  const f32x2_t v = {a, b};
  if constexpr (IO == DSA_DTYPE_BF16)
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
  else
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2_t));
}

template <int IO> __device__ __forceinline__ float to_f32(uint16_t h) {
  return IO == IO_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
}
template <int IO> __device__ __forceinline__ uint16_t from_f32(float f) {
  return IO == IO_BF16 ? f32_to_bf16_rne(f) : f32_to_f16_rne(f);
}

// Monotone map of a 16-bit float pattern (sign, magnitude m) to an unsigned key:
// 0x8000 + m for a positive value, 0x8000 - m for a negative one. Larger float ->
// larger key; +0 and -0 map to the same key 0x8000 (the goldens compare them equal),
// and no pattern maps to 0, which marks entries outside a row.
__device__ __forceinline__ uint32_t ord16(uint16_t h) {
  return (h & 0x8000u) ? (uint32_t)(uint16_t)(0x10000u - h) : (uint32_t)(h | 0x8000u);
}
// inverse of ord16 on keys 1..0xFFFF (0x8000 gives +0)
__device__ __forceinline__ uint16_t unord16(uint32_t k) {
  return (k & 0x8000u) ? (uint16_t)(k & 0x7FFFu) : (uint16_t)(0x10000u - k);
}

// ------------------------------------------------------------------ MFMA
template <int IO> struct Mfma;
template <> struct Mfma<IO_BF16> {
  static __device__ __forceinline__ f32x16 m32(uint4 a, uint4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 m16(uint4 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};
template <> struct Mfma<IO_F16> {
  static __device__ __forceinline__ f32x16 m32(uint4 a, uint4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 m16(uint4 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

// 32x32x16 MFMA chains with the accumulator in arch VGPRs. In a kernel whose other
// accumulators live in AGPRs the compiler selects the AGPR form for every builtin
// MFMA, so a short-lived accumulator would take AGPRs too (and its VALU reads one
// v_accvgpr_read each); written as inline asm, this one stays in VGPRs. The compiler
// does not see these as MFMAs, so the caller ends every chain with vacc_drain()
// before any VALU touches the accumulator or the chain's operand registers.
typedef int i32x4v __attribute__((ext_vector_type(4)));
template <int IO>
__device__ __forceinline__ f32x16 mfma32_vacc_first(uint4 a, uint4 b) {   // A B
  f32x16 c;
  const i32x4v av = __builtin_bit_cast(i32x4v, a), bv = __builtin_bit_cast(i32x4v, b);
  if constexpr (IO == IO_BF16)
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(c) : "v"(av), "v"(bv));
  else
    asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, 0" : "=&v"(c) : "v"(av), "v"(bv));
  return c;
}
template <int IO>
__device__ __forceinline__ void mfma32_vacc(f32x16& c, uint4 a, uint4 b) {   // c += A B
  const i32x4v av = __builtin_bit_cast(i32x4v, a), bv = __builtin_bit_cast(i32x4v, b);
  if constexpr (IO == IO_BF16)
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(av), "v"(bv));
  else
    asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+v"(c) : "v"(av), "v"(bv));
}
// Wait states after the last MFMA of a VGPR chain: an 8-pass XDL result read (or
// its operands overwritten) by VALU needs 11; 18 covers every XDL pass count.
__device__ __forceinline__ void vacc_drain(f32x16& c) { asm volatile("s_nop 15\n\ts_nop 1" : "+v"(c)); }
// The last step of a chain with its drain in the same statement: the compiler may copy
// the accumulator to other registers between two asm statements (a copy it places before
// a separate vacc_drain would read the MFMA's result in flight), never inside one.
template <int IO>
__device__ __forceinline__ void mfma32_vacc_last(f32x16& c, uint4 a, uint4 b) {   // c += A B, drained
  const i32x4v av = __builtin_bit_cast(i32x4v, a), bv = __builtin_bit_cast(i32x4v, b);
  if constexpr (IO == IO_BF16)
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0\n\ts_nop 15\n\ts_nop 1" : "+v"(c) : "v"(av), "v"(bv));
  else
    asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0\n\ts_nop 15\n\ts_nop 1" : "+v"(c) : "v"(av), "v"(bv));
}
// Same with the result in other registers than the accumulator read (c + A B, drained).
template <int IO>
__device__ __forceinline__ f32x16 mfma32_vacc_last_to(const f32x16& c, uint4 a, uint4 b) {
  f32x16 d;
  const i32x4v av = __builtin_bit_cast(i32x4v, a), bv = __builtin_bit_cast(i32x4v, b);
  if constexpr (IO == IO_BF16)
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %3\n\ts_nop 15\n\ts_nop 1" : "=&v"(d) : "v"(av), "v"(bv), "v"(c));
  else
    asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %3\n\ts_nop 15\n\ts_nop 1" : "=&v"(d) : "v"(av), "v"(bv), "v"(c));
  return d;
}

// Output layouts (CDNA3/CDNA4 MFMA, 64 lanes):
//  32x32: lane l, acc[r] (r < 16) holds C[row = (r/4)*8 + (l/32)*4 + r%4][col = l%32]
//  16x16: lane l, acc[r] (r < 4)  holds C[row = (l/16)*4 + r][col = l%16]
// Operands: lane l supplies 8 consecutive K values of A row (l%32 | l%16) and of
// B column (l%32 | l%16); the K group is l/32 (32x32x16) or l/16 (16x16x32).
__device__ __forceinline__ int m32_row(int r, int lane) { return (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3); }
__device__ __forceinline__ int m16_row(int r, int lane) { return (lane >> 4) * 4 + r; }

// ------------------------------------------------------------------ misc
// 16-byte load from global memory, addressed as such: a generic pointer can make the
// compiler emit flat loads (for instance where it turns `c ? load(p) : zero` into a
// load from a selected address), and a flat load is counted by lgkmcnt as well, so
// every later LDS wait would also wait for it.
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ldg16(const void* p) {
  return __builtin_bit_cast(uint4, *(const __attribute__((address_space(1))) u32x4v*)p);
}

// c ? ldg16(p) : zeros. Written with a plain vector type on purpose: `c ? ldg16(p) : z`
// with z a named uint4 (a class type) makes the compiler select between p and the
// address of a zero copy in scratch and issue one flat load from the result.
__device__ __forceinline__ uint4 ldg16_or0(bool c, const void* p) {
  u32x4v v = {0u, 0u, 0u, 0u};
  if (c) v = *(const __attribute__((address_space(1))) u32x4v*)p;
  return __builtin_bit_cast(uint4, v);
}

// Work-group barrier that orders LDS accesses only. __syncthreads() is a
// release/acquire fence on all address spaces, which makes every wave drain its
// outstanding global loads (vmcnt 0) at the barrier and so cancels any global
// prefetch issued before it; here only LDS traffic is waited for.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// 16-byte direct-to-LDS load: lane l writes LDS [lds_base + 16 l, +16). Issued
// as inline asm so the compiler does not track it: its wait insertion assumes
// every LDS read may alias an outstanding direct-to-LDS load and would drain
// the prefetched tiles (vmcnt 0) before each LDS read. Kernels using it order
// these loads themselves with wait_vmcnt and lds_barrier. An LDS DMA reading M0
// needs one wait state after the SALU write of M0 (the s_nop), and M0 is declared
// clobbered so the compiler keeps nothing of its own there across the statement.
__device__ __forceinline__ void lds_dma16_untracked(const void* gptr, void* lds_base) {
  const uint32_t m0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds_base;
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(gptr), "s"(m0) : "memory", "m0");
}

// Same with a wave-uniform base address (SGPR pair) and a per-lane 32-bit byte
// offset: lane l reads sbase + voff[l] and writes LDS [lds_base + 16 l, +16).
__device__ __forceinline__ void lds_dma16_sbase_untracked(const void* sbase, uint32_t voff, void* lds_base) {
  const uint32_t m0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds_base;
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(voff), "s"(sbase), "s"(m0) : "memory", "m0");
}

// x[l] + x[l ^ 32] on every lane, with one v_permlane32_swap (VALU, no LDS).
// After swapping the upper half of `a` with the lower half of `b` (both x),
// a[l] + b[l] = x[l mod 32] + x[l mod 32 + 32]. Written as inline asm with two
// distinct in/out registers: the compiler folds the builtin's two results of
// permlane32_swap(x, x) into one and returns 2 x[l]. The s_nop 1 gives the two
// wait states the swap needs after the VALU writes of its operands.
__device__ __forceinline__ float add_half_swap(float x) {
  float a = x, b = x;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return a + b;
}

// max(x[l], x[l ^ 32]) on every lane (same swap).
__device__ __forceinline__ float max_half_swap(float x) {
  float a = x, b = x;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return fmaxf(a, b);
}

// v_permlane32_swap: exchanges the upper half of `a` with the lower half of `b`,
// i.e. afterwards a[l + 32] = old b[l] and b[l] = old a[l + 32] for l < 32 (the
// other halves keep their values). Inline asm for the same reason as above; the
// s_nop 1 gives the wait states the swap needs after VALU writes of its operands.
__device__ __forceinline__ void swap_halves(uint32_t& a, uint32_t& b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}

// Wave-wide inclusive prefix sum / max over the 64 lanes with DPP, VALU only (the
// __shfl_* intrinsics lower to ds_bpermute: a dependent LDS round trip per step). Row
// shifts by 1, 2, 4, 8 scan each 16-lane row (lanes shifted in from outside the row
// read 0); row_bcast:15 then adds row 0's last lane to row 1 (and row 2's to row 3),
// row_bcast:31 adds lane 31 to rows 2 and 3. Unsigned max uses the same steps (0 is its
// identity).
// (OLD: the value lanes shifted in from outside a row, or rows the mask leaves out, read:
// the operation's identity)
template <int CTRL, int ROW_MASK, int OLD = 0>
__device__ __forceinline__ uint32_t dpp_shift(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(OLD, (int)x, CTRL, ROW_MASK, 0xF, false);
}
__device__ __forceinline__ uint32_t wave_incl_sum(uint32_t x) {
  x += dpp_shift<0x111, 0xF>(x);   // row_shr:1
  x += dpp_shift<0x112, 0xF>(x);   // row_shr:2
  x += dpp_shift<0x114, 0xF>(x);   // row_shr:4
  x += dpp_shift<0x118, 0xF>(x);   // row_shr:8
  x += dpp_shift<0x142, 0xA>(x);   // row_bcast:15 into rows 1, 3
  x += dpp_shift<0x143, 0xC>(x);   // row_bcast:31 into rows 2, 3
  return x;
}
// signed minimum (identity INT_MAX); lane 63 holds the wave's minimum
__device__ __forceinline__ int wave_incl_min_i32(int x) {
  constexpr int I = 0x7FFFFFFF;
  x = min(x, (int)dpp_shift<0x111, 0xF, I>((uint32_t)x));
  x = min(x, (int)dpp_shift<0x112, 0xF, I>((uint32_t)x));
  x = min(x, (int)dpp_shift<0x114, 0xF, I>((uint32_t)x));
  x = min(x, (int)dpp_shift<0x118, 0xF, I>((uint32_t)x));
  x = min(x, (int)dpp_shift<0x142, 0xA, I>((uint32_t)x));
  x = min(x, (int)dpp_shift<0x143, 0xC, I>((uint32_t)x));
  return x;
}
__device__ __forceinline__ uint32_t wave_incl_max(uint32_t x) {
  x = max(x, dpp_shift<0x111, 0xF>(x));
  x = max(x, dpp_shift<0x112, 0xF>(x));
  x = max(x, dpp_shift<0x114, 0xF>(x));
  x = max(x, dpp_shift<0x118, 0xF>(x));
  x = max(x, dpp_shift<0x142, 0xA>(x));
  x = max(x, dpp_shift<0x143, 0xC>(x));
  return x;
}

typedef short s16x4 __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16: 8 bytes per lane, transposed within groups of 16 lanes.
// With the address pattern of tr_frag below it yields an MFMA operand whose K
// runs down the rows of a row-major LDS array.
__device__ __forceinline__ uint2 ds_read_tr(const void* lds_ptr) {
  s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(const_cast<void*>(lds_ptr)));
  return __builtin_bit_cast(uint2, v);
}

// The same at a 32-bit LDS byte address (constant offsets added to it fold into the
// instruction's offset field).
__device__ __forceinline__ uint2 ds_read_tr_at(uint32_t lds_addr) {
  s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(uintptr_t)lds_addr);
  return __builtin_bit_cast(uint2, v);
}

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// s_waitcnt vmcnt(N) (gfx9 encoding; expcnt and lgkmcnt left unconstrained).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

__device__ __forceinline__ void stg16(void* p, uint4 v) { *reinterpret_cast<uint4*>(p) = v; }

__device__ __forceinline__ int batch_of_row(const int32_t* row_start, int batch, int r) {
  // largest b with row_start[b] <= r (row_start has batch+1 ascending entries)
  int lo = 0, hi = batch - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if (row_start[mid] <= r) lo = mid; else hi = mid - 1;
  }
  return lo;
}

}  // namespace dsa

// ------------------------------------------------------------------ launchers
// Host-side launch entry points implemented by each kernel translation unit
// and called by the C-ABI layer after argument validation.
struct LiScoreArgs {
  const void* q; const void* k; const void* w; int io; int wdt;
  const int32_t* row_start; const int32_t* key_start; const int32_t* act_q; const int32_t* act_k;
  int batch, total_rows, n1, n2, d, s2, max_rows_per_batch, max_kv, sparse_mode;
  uint16_t* scores; int64_t ld;
  // PA_BSND keys (block_table != nullptr): token t of batch b is row
  // block_table[b * max_blocks + t / page_bs] * page_bs + t % page_bs of `k`
  const int32_t* block_table = nullptr; int max_blocks = 0; int page_bs = 0; int64_t key_rows = 0;
  int key_split = 1;   // work-groups per row block, each over a share of its key tiles (set by the launcher)
};
constexpr int LI_MAX_BLOCKS = 8192;   // block-table row held in LDS by the paged score kernel
constexpr int LI_TOPK_MAX_K = 16384;  // top-k: the selected keys and their indices sorted in LDS
struct LiTopkArgs {
  const uint16_t* scores; int64_t ld; int io;
  const int32_t* row_start; const int32_t* act_q; const int32_t* act_k;
  int batch, total_rows, n2, s2, sparse_mode, k;
  int32_t* idx; uint16_t* val;
};
struct SfaArgs {
  const void* q; const void* qr; const void* k; const void* kr; int io;
  const int32_t* sidx; int topk; int sbs;
  const int32_t* block_table; int max_blocks; int page_bs;
  const int32_t* row_start; const int32_t* key_start; const int32_t* act_q; const int32_t* act_k;
  int batch, total_rows, n1, d, dr, s2; int64_t key_rows; int sparse_mode; float scale;
  void* out; float* sm_max; float* sm_sum;
  void* ws; size_t ws_bytes; int kv_splits;
  // teacher mode (the indexer KL losses): for query row r = b * t_s1 + s1 and its slot list,
  // t_p[r * t_ld + slot] = (1 / N1) sum_h exp(score - t_max[r N1 + h]) / (t_sum[r N1 + h] + 1e-8)
  float* t_p = nullptr; int t_ld = 0; const float* t_max = nullptr; const float* t_sum = nullptr; int t_s1 = 0;
};
hipError_t launch_li_score(const LiScoreArgs& a, hipStream_t s);
hipError_t launch_li_topk(const LiTopkArgs& a, hipStream_t s);
// sparse_count > LI_TOPK_MAX_K: every visible entry sorted in caller-provided scratch
size_t li_topk_workspace_bytes(int total_rows, int n2, int s2, int k);
hipError_t launch_li_topk_big(const LiTopkArgs& a, void* ws, hipStream_t s);
hipError_t launch_sfa_fwd(const SfaArgs& a, hipStream_t s);
// Teacher sums of the indexer KL losses on the attention kernel's S^T path (BSND keys
// [B, S2, 1, D | 64]): slot i of row r is key row b * S2 + clip(sidx[r][i], 0, S2 - 1) (slot i
// = key i when sidx is NULL), for the first min(topk, max(act_k - act_q + s1 + 1, 0)) slots;
// a.ws holds sfa_token_ws_bytes(total_rows, topk, 1) bytes. D in {128, 256, 512}, Dr = 64.
hipError_t launch_sfa_teacher(const SfaArgs& a, hipStream_t s);
size_t sfa_workspace_bytes(int total_rows, int n1, int d, int topk, int sbs, int kv_splits);
size_t sfa_workspace_zero_bytes();
// The library's static per-device workspace of DSA_SFA_NOALLOC_SCRATCH_BYTES (its
// address on the current device; its zero-row prefix cleared on first use)
hipError_t sfa_noalloc_workspace(hipStream_t s, void** ws);

// Per-row token lists (physical key rows in the golden's gather order,
// sparse_flash_attention_numpy.py:38-60) built by the forward's token-list
// kernels into a workspace of sfa_token_ws_bytes() bytes; shared with the
// backward pass.
struct SfaTokenLists {
  int32_t* counts;   // [rows]
  int32_t* tokens;   // [rows, tstride]
  int tstride;
};
size_t sfa_token_ws_bytes(int total_rows, int topk, int sbs);
hipError_t launch_sfa_token_lists(const SfaArgs& a, void* ws, SfaTokenLists* tl, hipStream_t s);

struct SfaBwdArgs {
  SfaArgs f;   // forward arguments (q, qr, k, kr, indices, lengths, shapes, scale)
  const void* d_out; const void* out; const float* sm_max; const float* sm_sum;
  void* dq; void* dqr; void* dk; void* dkr; void* dv;
  const int32_t* h_row_start; const int32_t* h_act_k;   // host copies (they size the library GEMMs)
};
// h_row_start [batch + 1] and h_act_k [batch]: host copies of the row offsets and kv
// lengths (they size the per-batch dense buffers)
size_t sfa_bwd_workspace_bytes(int batch, const int32_t* h_row_start, const int32_t* h_act_k, int s2,
                               int total_rows, int n1, int d, int topk, int sbs, int64_t key_rows);
hipError_t launch_sfa_bwd(const SfaBwdArgs& a, hipStream_t s);
// Why the backward's library GEMMs are unavailable (hipBLASLt failed to load), else ""
const char* sfa_bwd_library_error();

// sparse lightning-indexer grad KL loss (BSND)
// row stride of the sparse loss's per-key dI buffer (0: no key-major dKI pass)
int sli_km_sparse_ld(int rows, int topk, int s2, int didx);
size_t sli_grad_workspace_bytes(int rows, int topk, int64_t key_rows, int didx, int km_ld);
bool sli_grad_supported(int d, int dr, int nidx1, int didx, int topk);
hipError_t launch_sli_grad(const void* q, const void* k, const void* qr, const void* kr, const void* qi,
                           const void* ki, const void* w, int io, int wdt, const int32_t* sidx, int topk,
                           const float* sm_max, const float* sm_sum, const int32_t* act_q,
                           const int32_t* act_k, int batch, int s1, int s2, int n1, int d, int dr,
                           int nidx1, int didx, float scale, void* dqi, void* dki, void* dw, float* loss,
                           void* ws, hipStream_t s);
// dense lightning-indexer loss (BSND): every visible key is a slot; workspace as the
// sparse loss with topk = s2
bool dense_li_grad_supported(int n1, int n2, int d, int dr, int nidx1, int didx, int s2);
hipError_t launch_dense_li_lse(const void* qi, const void* ki, const void* w, int io, int wdt,
                               const int32_t* act_q, const int32_t* act_k, int batch, int s1, int s2,
                               int nidx1, int didx, float* out_max, float* out_sum, hipStream_t s);
hipError_t launch_dense_li_grad(const void* q, const void* k, const void* qr, const void* kr, const void* qi,
                                const void* ki, const void* w, int io, int wdt, const float* sm_max,
                                const float* sm_sum, const float* max_index, const float* sum_index,
                                const int32_t* act_q, const int32_t* act_k, int batch, int s1, int s2, int n1,
                                int n2, int d, int dr, int nidx1, int didx, float scale, void* dqi, void* dki,
                                void* dw, float* loss, void* ws, hipStream_t s);
