// C ABI of libdsa_mi355x.so: argument validation, error reporting, dispatch.
//
// Validation mirrors the ValueError conditions of the reference operators
// (lightning_indexer_triton.py:501-502, :524-525; sparse_flash_attention_triton.py
// :1341-1351, :1377-1378, :1391-1398) so a bad call fails here with a message
// instead of reaching a kernel; the Python layer raises the same conditions first.
#include <hip/hip_runtime.h>

#include <climits>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>

#include "../../include/dsa_mi355x.h"
#include "dsa_common.hpp"

bool li_score_supported_d(int d);

namespace {
thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) {
    g_err[0] = 0;
    return DSA_OK;
  }
  return fail(DSA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

bool is16(int dt) { return dt == DSA_DTYPE_BF16 || dt == DSA_DTYPE_F16; }
}  // namespace

extern "C" {

int dsa_abi_version(void) { return 1; }

const char* dsa_last_error(void) { return g_err; }

int dsa_li_score(const void* query, const void* key, const void* weights, int io_dtype,
                 int w_dtype, const int32_t* row_start, const int32_t* key_start,
                 const int32_t* act_q, const int32_t* act_k, int batch, int total_rows, int n1,
                 int n2, int d, int s2, int max_rows_per_batch, int max_kv, int sparse_mode,
                 uint16_t* scores, int64_t score_ld, void* stream) {
  if (!query || !key || !weights || !row_start || !key_start || !act_q || !act_k || !scores)
    return fail(DSA_ERR_INVALID, "dsa_li_score: null pointer argument");
  if (!is16(io_dtype)) return fail(DSA_ERR_INVALID, "dsa_li_score: io_dtype must be fp16 or bf16");
  if (!is16(w_dtype) && w_dtype != DSA_DTYPE_F32)
    return fail(DSA_ERR_INVALID, "dsa_li_score: weights dtype must be fp16, bf16 or fp32");
  if (batch <= 0 || total_rows < 0 || n1 <= 0 || n2 <= 0 || s2 < 0 || max_rows_per_batch < 0)
    return fail(DSA_ERR_INVALID, "dsa_li_score: non-positive shape");
  if (n1 % n2 != 0) return fail(DSA_ERR_INVALID, "N1(%d) must be divisible by N2(%d)", n1, n2);
  if (n1 / n2 > 128) return fail(DSA_ERR_UNSUPPORTED, "dsa_li_score: group size N1/N2=%d > 128", n1 / n2);
  if (!li_score_supported_d(d))
    return fail(DSA_ERR_UNSUPPORTED, "dsa_li_score: D=%d not in {64, 96, 128, 256, 512}", d);
  if (sparse_mode != 0 && sparse_mode != 3)
    return fail(DSA_ERR_INVALID, "dsa_li_score: sparse_mode must be 0 or 3");
  if (score_ld < s2) return fail(DSA_ERR_INVALID, "dsa_li_score: score_ld < S2");
  if (batch > 65535 || n2 > 65535) return fail(DSA_ERR_UNSUPPORTED, "dsa_li_score: batch or N2 > 65535");
  LiScoreArgs a{query, key, weights, io_dtype, w_dtype, row_start, key_start, act_q, act_k,
                batch, total_rows, n1, n2, d, s2, max_rows_per_batch, max_kv, sparse_mode,
                scores, score_ld};
  return hip_status(launch_li_score(a, (hipStream_t)stream), "dsa_li_score launch");
}

int dsa_li_score_paged(const void* query, const void* key_cache, const void* weights, int io_dtype,
                       int w_dtype, const int32_t* row_start, const int32_t* block_table,
                       int max_blocks, int page_block_size, int64_t key_rows, const int32_t* act_q,
                       const int32_t* act_k, int batch, int total_rows, int n1, int n2, int d,
                       int max_rows_per_batch, int max_kv, int sparse_mode, uint16_t* scores,
                       int64_t score_ld, void* stream) {
  if (!query || !key_cache || !weights || !row_start || !block_table || !act_q || !act_k || !scores)
    return fail(DSA_ERR_INVALID, "dsa_li_score_paged: null pointer argument");
  if (max_blocks <= 0 || page_block_size <= 0 || key_rows <= 0)
    return fail(DSA_ERR_INVALID, "dsa_li_score_paged: max_blocks, page_block_size and key_rows must be positive");
  if (max_blocks > LI_MAX_BLOCKS)
    return fail(DSA_ERR_UNSUPPORTED, "dsa_li_score_paged: max_blocks=%d > %d", max_blocks, LI_MAX_BLOCKS);
  const int64_t s2 = (int64_t)max_blocks * page_block_size;
  if (s2 > INT_MAX) return fail(DSA_ERR_UNSUPPORTED, "dsa_li_score_paged: max_blocks*block_size > 2^31-1");
  if (!is16(io_dtype)) return fail(DSA_ERR_INVALID, "dsa_li_score_paged: io_dtype must be fp16 or bf16");
  if (!is16(w_dtype) && w_dtype != DSA_DTYPE_F32)
    return fail(DSA_ERR_INVALID, "dsa_li_score_paged: weights dtype must be fp16, bf16 or fp32");
  if (batch <= 0 || total_rows < 0 || n1 <= 0 || n2 <= 0 || max_rows_per_batch < 0)
    return fail(DSA_ERR_INVALID, "dsa_li_score_paged: non-positive shape");
  if (n1 % n2 != 0) return fail(DSA_ERR_INVALID, "N1(%d) must be divisible by N2(%d)", n1, n2);
  if (n1 / n2 > 128) return fail(DSA_ERR_UNSUPPORTED, "dsa_li_score_paged: group size N1/N2=%d > 128", n1 / n2);
  if (!li_score_supported_d(d))
    return fail(DSA_ERR_UNSUPPORTED, "dsa_li_score_paged: D=%d not in {64, 96, 128, 256, 512}", d);
  if (sparse_mode != 0 && sparse_mode != 3)
    return fail(DSA_ERR_INVALID, "dsa_li_score_paged: sparse_mode must be 0 or 3");
  if (score_ld < s2) return fail(DSA_ERR_INVALID, "dsa_li_score_paged: score_ld < max_blocks*block_size");
  if (batch > 65535 || n2 > 65535) return fail(DSA_ERR_UNSUPPORTED, "dsa_li_score_paged: batch or N2 > 65535");
  LiScoreArgs a{query, key_cache, weights, io_dtype, w_dtype, row_start, act_q, act_q, act_k,
                batch, total_rows, n1, n2, d, (int)s2, max_rows_per_batch, max_kv, sparse_mode,
                scores, score_ld};
  a.block_table = block_table;
  a.max_blocks = max_blocks;
  a.page_bs = page_block_size;
  a.key_rows = key_rows;
  return hip_status(launch_li_score(a, (hipStream_t)stream), "dsa_li_score_paged launch");
}

namespace {
// Argument checks of dsa_li_topk / dsa_li_topk_ws; DSA_OK when the call may proceed.
int check_li_topk(const char* fn, const uint16_t* scores, int64_t score_ld, int io_dtype,
                  const int32_t* row_start, const int32_t* act_q, const int32_t* act_k, int batch,
                  int total_rows, int n2, int s2, int sparse_mode, int sparse_count, const int32_t* indices) {
  if (!scores || !row_start || !act_q || !act_k || !indices)
    return fail(DSA_ERR_INVALID, "%s: null pointer argument", fn);
  if (!is16(io_dtype)) return fail(DSA_ERR_INVALID, "%s: io_dtype must be fp16 or bf16", fn);
  if (batch <= 0 || total_rows < 0 || n2 <= 0 || s2 < 0)
    return fail(DSA_ERR_INVALID, "%s: non-positive shape", fn);
  if (sparse_count <= 0) return fail(DSA_ERR_INVALID, "%s: sparse_count must be positive", fn);
  if (sparse_mode != 0 && sparse_mode != 3)
    return fail(DSA_ERR_INVALID, "%s: sparse_mode must be 0 or 3", fn);
  if (score_ld < s2) return fail(DSA_ERR_INVALID, "%s: score_ld < S2", fn);
  return DSA_OK;
}
}  // namespace

int dsa_li_topk(const uint16_t* scores, int64_t score_ld, int io_dtype, const int32_t* row_start,
                const int32_t* act_q, const int32_t* act_k, int batch, int total_rows, int n2,
                int s2, int sparse_mode, int sparse_count, int32_t* indices, uint16_t* values,
                void* stream) {
  const int st = check_li_topk("dsa_li_topk", scores, score_ld, io_dtype, row_start, act_q, act_k, batch,
                               total_rows, n2, s2, sparse_mode, sparse_count, indices);
  if (st != DSA_OK) return st;
  if (sparse_count > LI_TOPK_MAX_K)
    return fail(DSA_ERR_UNSUPPORTED, "dsa_li_topk: sparse_count=%d > %d (use dsa_li_topk_ws)", sparse_count,
                LI_TOPK_MAX_K);
  LiTopkArgs a{scores, score_ld, io_dtype, row_start, act_q, act_k, batch, total_rows, n2, s2,
               sparse_mode, sparse_count, indices, values};
  return hip_status(launch_li_topk(a, (hipStream_t)stream), "dsa_li_topk launch");
}

size_t dsa_li_topk_workspace_bytes(int total_rows, int n2, int s2, int sparse_count) {
  return li_topk_workspace_bytes(total_rows, n2, s2, sparse_count);
}

int dsa_li_topk_ws(const uint16_t* scores, int64_t score_ld, int io_dtype, const int32_t* row_start,
                   const int32_t* act_q, const int32_t* act_k, int batch, int total_rows, int n2,
                   int s2, int sparse_mode, int sparse_count, int32_t* indices, uint16_t* values,
                   void* workspace, size_t workspace_bytes, void* stream) {
  const int st = check_li_topk("dsa_li_topk_ws", scores, score_ld, io_dtype, row_start, act_q, act_k, batch,
                               total_rows, n2, s2, sparse_mode, sparse_count, indices);
  if (st != DSA_OK) return st;
  LiTopkArgs a{scores, score_ld, io_dtype, row_start, act_q, act_k, batch, total_rows, n2, s2,
               sparse_mode, sparse_count, indices, values};
  if (sparse_count <= LI_TOPK_MAX_K)
    return hip_status(launch_li_topk(a, (hipStream_t)stream), "dsa_li_topk_ws launch");
  const size_t need = li_topk_workspace_bytes(total_rows, n2, s2, sparse_count);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return fail(DSA_ERR_INVALID, "dsa_li_topk_ws: workspace of %zu bytes < %zu", workspace_bytes, need);
  return hip_status(launch_li_topk_big(a, workspace, (hipStream_t)stream), "dsa_li_topk_ws launch");
}

size_t dsa_sfa_workspace_bytes(int total_rows, int n1, int d, int sparse_count,
                               int sparse_block_size, int kv_splits) {
  if (total_rows <= 0 || sparse_count <= 0 || sparse_block_size <= 0) return 0;
  return sfa_workspace_bytes(total_rows, n1, d, sparse_count, sparse_block_size, kv_splits);
}

size_t dsa_sfa_workspace_zero_bytes(void) { return sfa_workspace_zero_bytes(); }

namespace {
// Argument checks of dsa_sfa_fwd (the reference's conditions, sparse_flash_attention_triton.py
// :1341-1351, :1391-1398) shared with dsa_sfa_fwd_noalloc; DSA_OK when the call may proceed.
int check_sfa_fwd(const char* fn, const void* query, const void* query_rope, const void* key,
                  const void* key_rope, int io_dtype, const int32_t* sparse_indices, int sparse_count,
                  int sparse_block_size, const int32_t* block_table, int max_blocks, int page_block_size,
                  const int32_t* row_start, const int32_t* key_start, const int32_t* act_q,
                  const int32_t* act_k, int batch, int total_rows, int n1, int d, int dr, int64_t key_rows,
                  int sparse_mode, void* out, float* sm_max, float* sm_sum, int kv_splits) {
  if (!query || !query_rope || !key || !key_rope || !sparse_indices || !row_start || !act_q ||
      !act_k || !out)
    return fail(DSA_ERR_INVALID, "%s: null pointer argument", fn);
  if (!block_table && !key_start)
    return fail(DSA_ERR_INVALID, "%s: key_start required without block_table", fn);
  if (!is16(io_dtype)) return fail(DSA_ERR_INVALID, "%s: io_dtype must be fp16 or bf16", fn);
  if (sparse_mode != 0 && sparse_mode != 3)
    return fail(DSA_ERR_INVALID, "Only sparse_mode 0 (full) / 3 (rightDownCausal) supported");
  if (sparse_block_size < 1 || (sparse_block_size & (sparse_block_size - 1)) != 0 ||
      sparse_block_size > 128)
    return fail(DSA_ERR_INVALID, "sparse_block_size must be a power of 2 in [1,128]");
  if (d != 128 && d != 256 && d != 512)
    return fail(DSA_ERR_INVALID, "D must be one of (128, 256, 512), got %d", d);
  if (dr != 64) return fail(DSA_ERR_INVALID, "rope dim must be 64, got %d", dr);
  if (n1 < 1 || n1 > 128 || (n1 & (n1 - 1)) != 0)
    return fail(DSA_ERR_INVALID, "N1 must be one of (1, 2, 4, 8, 16, 32, 64, 128), got %d", n1);
  if (batch <= 0 || total_rows < 0 || sparse_count <= 0 || key_rows < 0)
    return fail(DSA_ERR_INVALID, "%s: non-positive shape", fn);
  if (block_table && (max_blocks <= 0 || page_block_size <= 0))
    return fail(DSA_ERR_INVALID, "%s: PA_BSND needs max_blocks and block_size > 0", fn);
  if ((sm_max == nullptr) != (sm_sum == nullptr))
    return fail(DSA_ERR_INVALID, "%s: sm_max and sm_sum must both be given or both NULL", fn);
  if ((int64_t)sparse_count * sparse_block_size > (1 << 20))
    return fail(DSA_ERR_UNSUPPORTED, "%s: sparse_count*sparse_block_size > 2^20 tokens", fn);
  if (kv_splits > 16) return fail(DSA_ERR_UNSUPPORTED, "%s: kv_splits=%d > 16", fn, kv_splits);
  return DSA_OK;
}
}  // namespace

int dsa_sfa_fwd_noalloc(const void* query, const void* query_rope, const void* key, const void* key_rope,
                        int io_dtype, const int32_t* sparse_indices, int sparse_count, int sparse_block_size,
                        const int32_t* block_table, int max_blocks, int page_block_size,
                        const int32_t* row_start, const int32_t* key_start, const int32_t* act_q,
                        const int32_t* act_k, int batch, int total_rows, int n1, int d, int dr, int s2,
                        int64_t key_rows, int sparse_mode, float scale, void* out, float* sm_max,
                        float* sm_sum, int kv_splits, void* stream) {
  const int st = check_sfa_fwd("dsa_sfa_fwd_noalloc", query, query_rope, key, key_rope, io_dtype,
                               sparse_indices, sparse_count, sparse_block_size, block_table, max_blocks,
                               page_block_size, row_start, key_start, act_q, act_k, batch, total_rows, n1,
                               d, dr, key_rows, sparse_mode, out, sm_max, sm_sum, kv_splits);
  if (st != DSA_OK) return st;
  if (total_rows == 0) {
    g_err[0] = 0;
    return DSA_OK;
  }
  const size_t need = sfa_workspace_bytes(total_rows, n1, d, sparse_count, sparse_block_size, kv_splits);
  if (need > DSA_SFA_NOALLOC_SCRATCH_BYTES)
    return fail(DSA_ERR_UNSUPPORTED,
                "dsa_sfa_fwd_noalloc: the problem needs %zu bytes of workspace, the static scratch holds %zu "
                "(use dsa_sfa_fwd with a caller workspace)", need, (size_t)DSA_SFA_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  const hipError_t e = sfa_noalloc_workspace((hipStream_t)stream, &ws);
  if (e != hipSuccess) return hip_status(e, "dsa_sfa_fwd_noalloc scratch set-up");
  SfaArgs a{query, query_rope, key, key_rope, io_dtype, sparse_indices, sparse_count,
            sparse_block_size, block_table, max_blocks, page_block_size, row_start, key_start,
            act_q, act_k, batch, total_rows, n1, d, dr, s2, key_rows, sparse_mode, scale, out, sm_max,
            sm_sum, ws, (size_t)DSA_SFA_NOALLOC_SCRATCH_BYTES, kv_splits};
  return hip_status(launch_sfa_fwd(a, (hipStream_t)stream), "dsa_sfa_fwd_noalloc launch");
}

int dsa_sfa_fwd(const void* query, const void* query_rope, const void* key, const void* key_rope,
                int io_dtype, const int32_t* sparse_indices, int sparse_count,
                int sparse_block_size, const int32_t* block_table, int max_blocks,
                int page_block_size, const int32_t* row_start, const int32_t* key_start,
                const int32_t* act_q, const int32_t* act_k, int batch, int total_rows, int n1,
                int d, int dr, int s2, int64_t key_rows, int sparse_mode, float scale, void* out,
                float* sm_max,
                float* sm_sum, void* workspace, size_t workspace_bytes, int kv_splits,
                void* stream) {
  const int st = check_sfa_fwd("dsa_sfa_fwd", query, query_rope, key, key_rope, io_dtype, sparse_indices,
                               sparse_count, sparse_block_size, block_table, max_blocks, page_block_size,
                               row_start, key_start, act_q, act_k, batch, total_rows, n1, d, dr, key_rows,
                               sparse_mode, out, sm_max, sm_sum, kv_splits);
  if (st != DSA_OK) return st;
  const size_t need = sfa_workspace_bytes(total_rows, n1, d, sparse_count, sparse_block_size, kv_splits);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return fail(DSA_ERR_INVALID, "dsa_sfa_fwd: workspace of %zu bytes required, %zu given", need,
                workspace_bytes);
  SfaArgs a{query, query_rope, key, key_rope, io_dtype, sparse_indices, sparse_count,
            sparse_block_size, block_table, max_blocks, page_block_size, row_start, key_start,
            act_q, act_k, batch, total_rows, n1, d, dr, s2, key_rows, sparse_mode, scale, out, sm_max,
            sm_sum, workspace, workspace_bytes, kv_splits};
  return hip_status(launch_sfa_fwd(a, (hipStream_t)stream), "dsa_sfa_fwd launch");
}

size_t dsa_sfa_bwd_workspace_bytes(int batch, const int32_t* host_row_start,
                                   const int32_t* host_act_k, int s2, int total_rows, int n1, int d,
                                   int sparse_count, int sparse_block_size, int64_t key_rows) {
  if (batch <= 0 || !host_row_start || !host_act_k || total_rows < 0 || n1 <= 0 || sparse_count <= 0 ||
      sparse_block_size <= 0 || key_rows < 0 || (d != 128 && d != 256 && d != 512))
    return 0;
  return sfa_bwd_workspace_bytes(batch, host_row_start, host_act_k, s2, total_rows, n1, d, sparse_count,
                                 sparse_block_size, key_rows);
}

int dsa_sfa_bwd(const void* query, const void* query_rope, const void* key, const void* key_rope,
                int io_dtype, const int32_t* sparse_indices, int sparse_count,
                int sparse_block_size, const int32_t* row_start, const int32_t* key_start,
                const int32_t* act_q, const int32_t* act_k, const int32_t* host_row_start,
                const int32_t* host_act_k, int batch, int total_rows, int n1, int d, int dr, int s2,
                int64_t key_rows, int sparse_mode, float scale, const void* d_out, const void* out,
                const float* sm_max, const float* sm_sum, void* d_query, void* d_query_rope,
                void* d_key, void* d_key_rope, void* d_value, void* workspace,
                size_t workspace_bytes, void* stream) {
  if (!query || !query_rope || !key || !key_rope || !sparse_indices || !row_start || !key_start ||
      !act_q || !act_k || !d_out || !out || !sm_max || !sm_sum || !d_query || !d_query_rope ||
      !d_key || !d_key_rope || !d_value || !workspace || !host_row_start || !host_act_k)
    return fail(DSA_ERR_INVALID, "dsa_sfa_bwd: null pointer argument");
  if (!is16(io_dtype)) return fail(DSA_ERR_INVALID, "dsa_sfa_bwd: io_dtype must be fp16 or bf16");
  if (sparse_mode != 0 && sparse_mode != 3)
    return fail(DSA_ERR_INVALID, "Only sparse_mode 0 (full) / 3 (rightDownCausal) supported");
  if (sparse_block_size < 1 || (sparse_block_size & (sparse_block_size - 1)) != 0 ||
      sparse_block_size > 128)
    return fail(DSA_ERR_INVALID, "sparse_block_size must be a power of 2 in [1,128]");
  if (d != 128 && d != 256 && d != 512)
    return fail(DSA_ERR_INVALID, "D must be one of (128, 256, 512), got %d", d);
  if (dr != 64) return fail(DSA_ERR_INVALID, "rope dim must be 64, got %d", dr);
  if (n1 < 1 || n1 > 128 || (n1 & (n1 - 1)) != 0)
    return fail(DSA_ERR_INVALID, "N1 must be one of (1, 2, 4, 8, 16, 32, 64, 128), got %d", n1);
  if (batch <= 0 || total_rows < 0 || sparse_count <= 0 || key_rows < 0)
    return fail(DSA_ERR_INVALID, "dsa_sfa_bwd: non-positive shape");
  if ((int64_t)sparse_count * sparse_block_size > (1 << 20))
    return fail(DSA_ERR_UNSUPPORTED, "dsa_sfa_bwd: sparse_count*sparse_block_size > 2^20 tokens");
  if (key_rows > INT32_MAX) return fail(DSA_ERR_UNSUPPORTED, "dsa_sfa_bwd: key_rows > 2^31-1");
  if (batch > 65535) return fail(DSA_ERR_UNSUPPORTED, "dsa_sfa_bwd: batch > 65535");
  if (host_row_start[0] != 0 || host_row_start[batch] > total_rows)
    return fail(DSA_ERR_INVALID, "dsa_sfa_bwd: host_row_start must start at 0 and end within total_rows");
  for (int b = 0; b < batch; ++b)   // the host copies size and place the library GEMMs
    if (host_row_start[b + 1] < host_row_start[b])
      return fail(DSA_ERR_INVALID, "dsa_sfa_bwd: host_row_start must be non-decreasing");
  const size_t need = sfa_bwd_workspace_bytes(batch, host_row_start, host_act_k, s2, total_rows, n1, d,
                                              sparse_count, sparse_block_size, key_rows);
  if (workspace_bytes < need)
    return fail(DSA_ERR_INVALID, "dsa_sfa_bwd: workspace of %zu bytes required, %zu given", need,
                workspace_bytes);
  SfaBwdArgs a{};
  a.f = SfaArgs{query, query_rope, key, key_rope, io_dtype, sparse_indices, sparse_count,
                sparse_block_size, nullptr, 0, 0, row_start, key_start, act_q, act_k, batch,
                total_rows, n1, d, dr, s2, key_rows, sparse_mode, scale, nullptr, nullptr, nullptr,
                workspace, workspace_bytes, 1};
  a.d_out = d_out;
  a.out = out;
  a.sm_max = sm_max;
  a.sm_sum = sm_sum;
  a.dq = d_query;
  a.dqr = d_query_rope;
  a.dk = d_key;
  a.dkr = d_key_rope;
  a.dv = d_value;
  a.h_row_start = host_row_start;
  a.h_act_k = host_act_k;
  const hipError_t e = launch_sfa_bwd(a, (hipStream_t)stream);
  if (e == hipErrorSharedObjectInitFailed)
    return fail(DSA_ERR_UNSUPPORTED, "dsa_sfa_bwd: %s", sfa_bwd_library_error());
  if (e == hipErrorStreamCaptureUnsupported)
    return fail(DSA_ERR_UNSUPPORTED,
                "dsa_sfa_bwd: the first call on a device creates its hipBLASLt handle and must run "
                "outside stream capture");
  return hip_status(e, "dsa_sfa_bwd launch");
}

size_t dsa_sli_grad_workspace_bytes(int batch, int s1, int s2, int sparse_count, int d_idx) {
  if (batch <= 0 || s1 < 0 || s2 <= 0 || sparse_count <= 0 || d_idx <= 0) return 0;
  return sli_grad_workspace_bytes(batch * s1, sparse_count, (int64_t)batch * s2, d_idx,
                                  sli_km_sparse_ld(batch * s1, sparse_count, s2, d_idx));
}

int dsa_sli_grad_kl_loss(const void* query, const void* key, const void* query_rope, const void* key_rope,
                         const void* query_index, const void* key_index, const void* weights, int io_dtype,
                         int w_dtype, const int32_t* sparse_indices, int sparse_count, const float* sm_max,
                         const float* sm_sum, const int32_t* act_q, const int32_t* act_k, int batch, int s1,
                         int s2, int n1, int d, int dr, int nidx1, int d_idx, float scale,
                         void* d_query_index, void* d_key_index, void* d_weights, float* loss,
                         void* workspace, size_t workspace_bytes, void* stream) {
  if (!query || !key || !query_index || !key_index || !weights || !sparse_indices || !sm_max || !sm_sum ||
      !act_q || !act_k || !d_query_index || !d_key_index || !d_weights || !loss || !workspace ||
      (dr > 0 && (!query_rope || !key_rope)))
    return fail(DSA_ERR_INVALID, "dsa_sli_grad_kl_loss: null pointer argument");
  if (!is16(io_dtype)) return fail(DSA_ERR_INVALID, "dsa_sli_grad_kl_loss: io_dtype must be fp16 or bf16");
  if (!is16(w_dtype) && w_dtype != DSA_DTYPE_F32)
    return fail(DSA_ERR_INVALID, "dsa_sli_grad_kl_loss: weights dtype must be fp16, bf16 or fp32");
  if (batch <= 0 || s1 < 0 || s2 <= 0 || n1 <= 0 || sparse_count <= 0)
    return fail(DSA_ERR_INVALID, "dsa_sli_grad_kl_loss: non-positive shape");
  if (n1 > 128) return fail(DSA_ERR_UNSUPPORTED, "dsa_sli_grad_kl_loss: N1=%d > 128", n1);
  if (dr != 0 && dr != 64) return fail(DSA_ERR_INVALID, "rope dim must be 64 (or 0 without rope), got %d", dr);
  if (!sli_grad_supported(d, dr, nidx1, d_idx, sparse_count))
    return fail(DSA_ERR_UNSUPPORTED,
                "dsa_sli_grad_kl_loss: D=%d (+%d), Nidx1=%d, D_idx=%d, topK=%d outside D in {128,256,512}, "
                "D_idx in {128,256,512}, Nidx1 <= 128, topK <= 2048",
                d, dr, nidx1, d_idx, sparse_count);
  if (batch > 65535 || (int64_t)batch * s1 > INT32_MAX)
    return fail(DSA_ERR_UNSUPPORTED, "dsa_sli_grad_kl_loss: too many rows");
  const size_t need = sli_grad_workspace_bytes(batch * s1, sparse_count, (int64_t)batch * s2, d_idx,
                                               sli_km_sparse_ld(batch * s1, sparse_count, s2, d_idx));
  if (workspace_bytes < need)
    return fail(DSA_ERR_INVALID, "dsa_sli_grad_kl_loss: workspace of %zu bytes required, %zu given", need,
                workspace_bytes);
  if (batch * s1 == 0) return DSA_OK;
  return hip_status(launch_sli_grad(query, key, query_rope ? query_rope : query, key_rope ? key_rope : key,
                                    query_index, key_index, weights, io_dtype, w_dtype, sparse_indices,
                                    sparse_count, sm_max, sm_sum, act_q, act_k, batch, s1, s2, n1, d, dr,
                                    nidx1, d_idx, scale, d_query_index, d_key_index, d_weights, loss,
                                    workspace, (hipStream_t)stream),
                    "dsa_sli_grad_kl_loss launch");
}

size_t dsa_dense_li_grad_workspace_bytes(int batch, int s1, int s2, int d_idx) {
  if (batch <= 0 || s1 < 0 || s2 <= 0 || d_idx <= 0) return 0;
  return sli_grad_workspace_bytes(batch * s1, s2, (int64_t)batch * s2, d_idx, 0);
}

int dsa_dense_li_softmax_lse(const void* query_index, const void* key_index, const void* weights, int io_dtype,
                             int w_dtype, const int32_t* act_q, const int32_t* act_k, int batch, int s1, int s2,
                             int nidx1, int d_idx, float* softmax_max_index, float* softmax_sum_index,
                             void* stream) {
  if (!query_index || !key_index || !weights || !act_q || !act_k || !softmax_max_index || !softmax_sum_index)
    return fail(DSA_ERR_INVALID, "dsa_dense_li_softmax_lse: null pointer argument");
  if (!is16(io_dtype)) return fail(DSA_ERR_INVALID, "dsa_dense_li_softmax_lse: io_dtype must be fp16 or bf16");
  if (!is16(w_dtype) && w_dtype != DSA_DTYPE_F32)
    return fail(DSA_ERR_INVALID, "dsa_dense_li_softmax_lse: weights dtype must be fp16, bf16 or fp32");
  if (batch <= 0 || s1 < 0 || s2 <= 0) return fail(DSA_ERR_INVALID, "dsa_dense_li_softmax_lse: non-positive shape");
  if (!dense_li_grad_supported(1, 1, 128, 0, nidx1, d_idx, s2))
    return fail(DSA_ERR_UNSUPPORTED,
                "dsa_dense_li_softmax_lse: Nidx1=%d, D_idx=%d outside D_idx in {128,256,512}, Nidx1 <= 128",
                nidx1, d_idx);
  if (batch > 65535 || (int64_t)batch * s1 > INT32_MAX)
    return fail(DSA_ERR_UNSUPPORTED, "dsa_dense_li_softmax_lse: too many rows");
  if (batch * s1 == 0) return DSA_OK;
  return hip_status(launch_dense_li_lse(query_index, key_index, weights, io_dtype, w_dtype, act_q, act_k, batch,
                                        s1, s2, nidx1, d_idx, softmax_max_index, softmax_sum_index,
                                        (hipStream_t)stream),
                    "dsa_dense_li_softmax_lse launch");
}

int dsa_dense_li_grad_kl_loss(const void* query, const void* key, const void* query_rope, const void* key_rope,
                              const void* query_index, const void* key_index, const void* weights, int io_dtype,
                              int w_dtype, const float* sm_max, const float* sm_sum, const float* max_index,
                              const float* sum_index, const int32_t* act_q, const int32_t* act_k, int batch,
                              int s1, int s2, int n1, int n2, int d, int dr, int nidx1, int d_idx, float scale,
                              void* d_query_index, void* d_key_index, void* d_weights, float* loss,
                              void* workspace, size_t workspace_bytes, void* stream) {
  if (!query || !key || !query_index || !key_index || !weights || !sm_max || !sm_sum || !act_q || !act_k ||
      !d_query_index || !d_key_index || !d_weights || !loss || !workspace ||
      (dr > 0 && (!query_rope || !key_rope)) || (!max_index != !sum_index))
    return fail(DSA_ERR_INVALID, "dsa_dense_li_grad_kl_loss: null pointer argument");
  if (!is16(io_dtype)) return fail(DSA_ERR_INVALID, "dsa_dense_li_grad_kl_loss: io_dtype must be fp16 or bf16");
  if (!is16(w_dtype) && w_dtype != DSA_DTYPE_F32)
    return fail(DSA_ERR_INVALID, "dsa_dense_li_grad_kl_loss: weights dtype must be fp16, bf16 or fp32");
  if (batch <= 0 || s1 < 0 || s2 <= 0 || n1 <= 0 || n2 <= 0)
    return fail(DSA_ERR_INVALID, "dsa_dense_li_grad_kl_loss: non-positive shape");
  if (n1 % n2 != 0) return fail(DSA_ERR_INVALID, "dsa_dense_li_grad_kl_loss: N1=%d not divisible by N2=%d", n1, n2);
  if (n1 > 128) return fail(DSA_ERR_UNSUPPORTED, "dsa_dense_li_grad_kl_loss: N1=%d > 128", n1);
  if (dr != 0 && dr != 64) return fail(DSA_ERR_INVALID, "rope dim must be 64 (or 0 without rope), got %d", dr);
  if (!dense_li_grad_supported(n1, n2, d, dr, nidx1, d_idx, s2))
    return fail(DSA_ERR_UNSUPPORTED,
                "dsa_dense_li_grad_kl_loss: D=%d (+%d), N1=%d, N2=%d, Nidx1=%d, D_idx=%d outside D, D_idx in "
                "{128,256,512}, Nidx1 <= 128", d, dr, n1, n2, nidx1, d_idx);
  if (batch > 65535 || (int64_t)batch * s1 > INT32_MAX)
    return fail(DSA_ERR_UNSUPPORTED, "dsa_dense_li_grad_kl_loss: too many rows");
  const size_t need = sli_grad_workspace_bytes(batch * s1, s2, (int64_t)batch * s2, d_idx, 0);
  if (workspace_bytes < need)
    return fail(DSA_ERR_INVALID, "dsa_dense_li_grad_kl_loss: workspace of %zu bytes required, %zu given", need,
                workspace_bytes);
  if (batch * s1 == 0) return DSA_OK;
  return hip_status(launch_dense_li_grad(query, key, query_rope ? query_rope : query, key_rope ? key_rope : key,
                                         query_index, key_index, weights, io_dtype, w_dtype, sm_max, sm_sum,
                                         max_index, sum_index, act_q, act_k, batch, s1, s2, n1, n2, d, dr, nidx1,
                                         d_idx, scale, d_query_index, d_key_index, d_weights, loss, workspace,
                                         (hipStream_t)stream),
                    "dsa_dense_li_grad_kl_loss launch");
}

}  // extern "C"
