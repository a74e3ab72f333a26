/*
 * dsa_mi355x.h — C ABI of the MI355X (gfx950) DeepSeek-Sparse-Attention hot path.
 *
 * The reference binds its device work through two MindSpore `_ms_pyfunc`
 * cores plus a library top-k; each entry point below replaces one of them:
 *
 *   dsa_li_score   <- _lightning_indexer_score_core   lightning_indexer_triton.py:386-417
 *                     (+ _lightning_indexer_score_kernel :180-284)
 *   dsa_li_topk    <- _stable_topk                     lightning_indexer_triton.py:343-361
 *                     with the golden's ordering       lightning_indexer_numpy.py:92-105
 *   dsa_sfa_fwd    <- _sfa_core                        sparse_flash_attention_triton.py:1160-1289
 *                     (+ _sfa_kernel :324-604, _sfa_gather_kernel :611-679,
 *                        _sfa_kernel_gathered :710-962, _pa_to_bsnd :1012-1033,
 *                        _expand_block_indices :1036-1051)
 *   dsa_sfa_workspace_bytes <- the workspace sizing of _sfa_core :1218-1250
 *                     (the caller allocates; the library keeps no cache)
 *   dsa_sfa_bwd    <- _sfa_grad_core                   sparse_flash_attention_grad_triton.py:441-495
 *                     (+ _sfa_grad_kernel :157-415)
 *   dsa_li_score_paged: dsa_li_score over a paged key cache (an extension; the
 *                     reference's indexer rejects block_table)
 *
 * Conventions
 *  - Every pointer is device memory unless stated; the caller owns every buffer.
 *  - `stream` is a hipStream_t passed as void* (NULL = the null stream). Calls
 *    are asynchronous on that stream.
 *  - Return 0 on success, DSA_ERR_* (< 0) otherwise; dsa_last_error() gives a
 *    thread-local message for the last failing call on the calling thread.
 *  - Query rows are "packed rows": BSND row r = b*S1 + s1, TND row r = cu_q[b-1] + s1.
 *    row_start[B+1] gives the first packed row of each batch (BSND: b*S1,
 *    TND: 0, cu_q[0], ...); key_start[B] the first packed key row (BSND: b*S2,
 *    TND: 0, cu_k[0], ...). act_q / act_k are per-batch lengths.
 */
#ifndef DSA_MI355X_H
#define DSA_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DSA_DTYPE_F16 0
#define DSA_DTYPE_BF16 1
#define DSA_DTYPE_F32 2

#define DSA_OK 0
#define DSA_ERR_INVALID (-1)     /* argument outside the documented domain */
#define DSA_ERR_UNSUPPORTED (-2) /* valid for the reference, not implemented here */
#define DSA_ERR_HIP (-3)         /* a HIP runtime call failed */

/* ABI version of this header (bumped on any signature change). */
int dsa_abi_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char* dsa_last_error(void);

/*
 * Indexer scores (replaces _lightning_indexer_score_core,
 * lightning_indexer_triton.py:386-417).
 *
 *   score[r*N2+n2, s2] = sum_{g < G} relu(q[r, n2*G+g, :] . k[key_start[b]+s2, n2, :]) * w[r, n2*G+g]
 *
 * quantised to the io dtype (bf16 RNE / fp16) and written as 16-bit patterns to
 * scores[(r*N2+n2)*score_ld + s2] for the visible prefix s2 < L(r) only, where
 * L = min(max(act_k-act_q+s1+1, 0), S2, act_k) for sparse_mode 3 and
 * min(act_k, S2) for sparse_mode 0 (lightning_indexer_numpy.py:85-90).
 * Rows with s1 >= act_q[b] are not written.
 *   query  [total_rows, N1, D] io dtype;  key [.., N2, D] io dtype;
 *   weights[total_rows, N1] in w_dtype (fp16 / bf16 / fp32);
 *   io_dtype DSA_DTYPE_BF16 or DSA_DTYPE_F16;  D in {64, 96, 128, 256, 512};
 *   N1 % N2 == 0;  sparse_mode 0 or 3;  score_ld >= S2.
 *   max_rows_per_batch = max_b(row_start[b+1]-row_start[b]) (host-known bound);
 *   max_kv = max_b act_k[b] (host-known bound, <= S2).
 */
int dsa_li_score(const void* query, const void* key, const void* weights, int io_dtype,
                 int w_dtype, const int32_t* row_start, const int32_t* key_start,
                 const int32_t* act_q, const int32_t* act_k, int batch, int total_rows, int n1,
                 int n2, int d, int s2, int max_rows_per_batch, int max_kv, int sparse_mode,
                 uint16_t* scores, int64_t score_ld, void* stream);

/*
 * dsa_li_score with the keys in a paged cache (PA_BSND). No counterpart in the
 * reference: lightning_indexer_triton rejects block_table (:501-502); the
 * semantics are those of dsa_li_score on the keys de-paged the way the reference
 * de-pages the SFA cache (_pa_to_bsnd, sparse_flash_attention_triton.py:1012-1033).
 *   key_cache [num_blocks, page_block_size, N2, D]; key_rows = num_blocks * page_block_size;
 *   block_table [batch, max_blocks] int32: token t of batch b is cache row
 *     block_table[b*max_blocks + t/page_block_size]*page_block_size + t%page_block_size;
 *     a -1 block (or one past the cache) is a zero key row: its scores are 0.
 *   S2 = max_blocks * page_block_size (max_blocks <= 8192); score_ld >= S2.
 * Everything else as dsa_li_score (act_k[b] keys visible; no key_start).
 */
int dsa_li_score_paged(const void* query, const void* key_cache, const void* weights, int io_dtype,
                       int w_dtype, const int32_t* row_start, const int32_t* block_table,
                       int max_blocks, int page_block_size, int64_t key_rows, const int32_t* act_q,
                       const int32_t* act_k, int batch, int total_rows, int n1, int n2, int d,
                       int max_rows_per_batch, int max_kv, int sparse_mode, uint16_t* scores,
                       int64_t score_ld, void* stream);

/*
 * Stable top-k over the quantised score rows (replaces _stable_topk,
 * lightning_indexer_triton.py:343-361, with the golden's order,
 * lightning_indexer_numpy.py:92-105): per score row, entries of the visible
 * prefix ordered by score descending then index ascending; the first
 * min(L, sparse_count) are written to indices[(r*N2+n2)*sparse_count + i]
 * (int32) and, if `values` is not NULL, their 16-bit score to values[...];
 * the remaining slots get index -1 and value 0. Rows with s1 >= act_q are all -1 / 0.
 * Scores compare as the floats their bit patterns encode, with +0 == -0 (a -0 is
 * returned as +0); NaN patterns, which the golden's contract excludes, order by their
 * bits: negative ones below -inf, positive ones above +inf.
 * Any S2 (int32 indices); sparse_count <= 16384 (DSA_ERR_UNSUPPORTED above: use
 * dsa_li_topk_ws).
 */
int dsa_li_topk(const uint16_t* scores, int64_t score_ld, int io_dtype,
                const int32_t* row_start, const int32_t* act_q, const int32_t* act_k,
                int batch, int total_rows, int n2, int s2, int sparse_mode, int sparse_count,
                int32_t* indices, uint16_t* values, void* stream);

/*
 * Bytes of device workspace dsa_li_topk_ws needs: 0 for sparse_count <= 16384, else two
 * buffers of S2 8-byte entries per score row (total_rows * N2 * 16 * S2).
 */
size_t dsa_li_topk_workspace_bytes(int total_rows, int n2, int s2, int sparse_count);

/*
 * dsa_li_topk for any sparse_count (the reference's _stable_topk,
 * lightning_indexer_triton.py:343-361, has no cap): sparse_count <= 16384 runs
 * dsa_li_topk's kernel and ignores the workspace; above, every visible entry of a row
 * is sorted (stable, score descending) in `workspace`, which must hold
 * dsa_li_topk_workspace_bytes (DSA_ERR_INVALID otherwise). Same outputs and ordering.
 */
int dsa_li_topk_ws(const uint16_t* scores, int64_t score_ld, int io_dtype,
                   const int32_t* row_start, const int32_t* act_q, const int32_t* act_k,
                   int batch, int total_rows, int n2, int s2, int sparse_mode, int sparse_count,
                   int32_t* indices, uint16_t* values, void* workspace, size_t workspace_bytes,
                   void* stream);

/*
 * Bytes of device workspace dsa_sfa_fwd needs for this problem (token lists and,
 * for KV-split rows, the split partials). kv_splits <= 0 selects the library's choice.
 */
size_t dsa_sfa_workspace_bytes(int total_rows, int n1, int d, int sparse_count,
                               int sparse_block_size, int kv_splits);

/*
 * Bytes at the start of every dsa_sfa_fwd workspace that must be zero when the
 * workspace is first used (the zero KV row; no call writes anything but zeros
 * there). The rest of the workspace needs no initialisation. No counterpart in the
 * reference (its workspace cache is internal, sparse_flash_attention_triton.py:37).
 */
size_t dsa_sfa_workspace_zero_bytes(void);

/*
 * Sparse flash attention forward, MLA-absorb (replaces _sfa_core,
 * sparse_flash_attention_triton.py:1160-1289; semantics of
 * sparse_flash_attention_numpy.py:38-160).
 *
 * For each packed query row r (batch b, s1 = r - row_start[b], s1 < act_q[b]):
 *   threshold = act_k (mode 0) | act_k - act_q + s1 + 1 (mode 3; rows with
 *   s1 < act_q - act_k are skipped); the first min(count, ceil(threshold/bs))
 *   ids of sparse_indices[r, :] are scanned, stopping at the first -1; id i
 *   expands to tokens [i*bs, min(i*bs+bs, act_k, threshold)).
 *   score[h, t] = (q[r,h,:D].k[t,:D] + q_rope[r,h,:].k_rope[t,:]) * scale
 *   out[r, h, :] = softmax_t(score[h, :]) @ k[t, :D]       (value = key)
 *   sm_max[r*N1+h] = max_t score,  sm_sum[r*N1+h] = sum_t exp(score - max)
 * Skipped rows / rows without tokens get out = 0, sm = 0.
 *
 *   query [total_rows, N1, D], query_rope [total_rows, N1, Dr], io dtype;
 *   key / key_rope: BSND or TND [.., 1, D|Dr] with token t at row key_start[b]+t,
 *     or PA_BSND [num_blocks, page_block_size, 1, D|Dr] when block_table != NULL:
 *     token t of batch b lives in block block_table[b*max_blocks + t/page_block_size]
 *     (-1 block -> a zero row, like the reference's de-paging);
 *   sparse_indices [total_rows, sparse_count] int32 block ids;
 *   key_rows: rows held by key / key_rope (num_blocks*page_block_size for PA_BSND);
 *     a gathered token outside [0, key_rows) reads as a zero row (never out of bounds).
 *   N1 <= 128, D in {128, 256, 512}, Dr = 64, sparse_block_size a power of 2 <= 128.
 *   sm_max / sm_sum may be NULL (not requested).
 *   workspace: >= dsa_sfa_workspace_bytes(...) bytes whose first
 *     dsa_sfa_workspace_zero_bytes() bytes are zero before its first use (e.g. one
 *     hipMemset at allocation): they hold a zero KV row that no call overwrites with
 *     anything but zeros, so they are cleared once, not per call.
 *     Calls that share a workspace must be ordered (same stream or synchronised).
 *   kv_splits: KV splits per row (<= 0: the library's choice, at most 16). Several
 *     splits add a merge launch; with sparse_block_size 1 the splits list their own
 *     tokens (no token-list launch).
 */
int dsa_sfa_fwd(const void* query, const void* query_rope, const void* key,
                const void* key_rope, int io_dtype, const int32_t* sparse_indices,
                int sparse_count, int sparse_block_size, const int32_t* block_table,
                int max_blocks, int page_block_size, const int32_t* row_start,
                const int32_t* key_start, const int32_t* act_q, const int32_t* act_k, int batch,
                int total_rows, int n1, int d, int dr, int s2, int64_t key_rows, int sparse_mode,
                float scale,
                void* out, float* sm_max, float* sm_sum, void* workspace,
                size_t workspace_bytes, int kv_splits, void* stream);

/*
 * dsa_sfa_fwd without a caller workspace. No counterpart in the reference: for callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). Arguments, semantics and outputs are those
 * of dsa_sfa_fwd (same kernels); the workspace is the library's static per-device
 * scratch array of DSA_SFA_NOALLOC_SCRATCH_BYTES (40 MiB), part of the library's code
 * object: every process that loads the library holds it on every GPU where the module is
 * loaded, until the process ends, whether or not it calls this entry point. A problem
 * whose dsa_sfa_workspace_bytes(...) exceeds that size is refused with
 * DSA_ERR_UNSUPPORTED before any device work (C4 decode, 64 rows x 2048 tokens: 32.9 MiB,
 * and C3 prefill, 4096 rows x 2048 tokens: 32.0 MiB, fit). The call
 * allocates nothing; its first call on a device looks up that device's copy of the
 * array and clears its zero-row prefix once (synchronising the given stream unless it
 * is capturing). Every call on one GPU shares that GPU's array: calls that overlap on
 * one GPU (different streams, or host threads without ordering) race and must be
 * serialised by the caller.
 */
#define DSA_SFA_NOALLOC_SCRATCH_BYTES ((size_t)40 << 20)

int dsa_sfa_fwd_noalloc(const void* query, const void* query_rope, const void* key,
                        const void* key_rope, int io_dtype, const int32_t* sparse_indices,
                        int sparse_count, int sparse_block_size, const int32_t* block_table,
                        int max_blocks, int page_block_size, const int32_t* row_start,
                        const int32_t* key_start, const int32_t* act_q, const int32_t* act_k,
                        int batch, int total_rows, int n1, int d, int dr, int s2, int64_t key_rows,
                        int sparse_mode, float scale, void* out, float* sm_max, float* sm_sum,
                        int kv_splits, void* stream);

/*
 * Workspace bytes for dsa_sfa_bwd: the token lists of total_rows rows, a staging
 * area of 4 fp32 partials of sum_b min(act_k[b], s2) rows of [d_key | d_key_rope |
 * d_value],
 * a [total_rows * N1, D + 64] copy of [query | query_rope], 128 MiB for the library
 * GEMMs, and two dense io-dtype buffers of sum_b min(act_k[b], s2) * ceil64(rows_b *
 * N1) elements (rows_b = host_row_start[b+1] - host_row_start[b]). host_row_start [batch + 1] and
 * host_act_k [batch] are host copies of the row offsets and kv lengths. Needs no
 * initialisation. No counterpart in the reference (it allocates its buffers per
 * call, sparse_flash_attention_grad_triton.py:634-642).
 */
size_t dsa_sfa_bwd_workspace_bytes(int batch, const int32_t* host_row_start,
                                   const int32_t* host_act_k, int s2, int total_rows, int n1, int d,
                                   int sparse_count, int sparse_block_size, int64_t key_rows);

/*
 * Sparse flash attention backward, MLA-absorb (replaces _sfa_grad_core,
 * sparse_flash_attention_grad_triton.py:441-495; semantics of
 * sparse_flash_attention_grad_numpy.py:34-143).
 *
 * Rows, tokens, shapes and layouts as dsa_sfa_fwd (no block table). With the
 * forward's out and its softmax stats (sm_max / sm_sum, [total_rows * N1] fp32):
 *   P[h, t]  = exp(score[h, t] - sm_max) / sm_sum
 *   dS[h, t] = P * (d_out[r,h,:].k[t,:D] - d_out[r,h,:].out[r,h,:]) * scale
 *   d_query[r,h,:] = sum_t dS k[t,:D],   d_query_rope[r,h,:] = sum_t dS k_rope[t,:]
 *   d_key[t,:]  += sum_h dS q[r,h,:],    d_key_rope[t,:] += sum_h dS q_rope[r,h,:]
 *   d_value[t,:] += sum_h P d_out[r,h,:]   (summed over every row selecting t)
 * d_query / d_query_rope are [total_rows, N1, D|Dr]; d_key / d_key_rope / d_value are
 * [key_rows, D|Dr] over the whole key tensors (rows no query selects are zero); all in
 * the io dtype, accumulated in fp32. The order of the fp32 additions into a key row is
 * not fixed (the reference's deterministic=False contract). Key token t of batch b is
 * key row key_start[b] + t for t < min(act_k[b], s2).
 *   host_row_start / host_act_k: host copies of row_start / act_k (same values).
 *   workspace: >= dsa_sfa_bwd_workspace_bytes(...) bytes; calls sharing it must be
 *   ordered on one stream.
 */
int dsa_sfa_bwd(const void* query, const void* query_rope, const void* key, const void* key_rope,
                int io_dtype, const int32_t* sparse_indices, int sparse_count,
                int sparse_block_size, const int32_t* row_start, const int32_t* key_start,
                const int32_t* act_q, const int32_t* act_k, const int32_t* host_row_start,
                const int32_t* host_act_k, int batch, int total_rows, int n1, int d, int dr, int s2,
                int64_t key_rows, int sparse_mode, float scale, const void* d_out, const void* out,
                const float* sm_max, const float* sm_sum, void* d_query, void* d_query_rope,
                void* d_key, void* d_key_rope, void* d_value, void* workspace,
                size_t workspace_bytes, void* stream);

/*
 * Workspace bytes for dsa_sli_grad_kl_loss: fp32 teacher sums [batch*s1, sparse_count],
 * an fp32 d_key_index accumulator [batch*s2, d_idx], for d_idx = 128 with s2 <= 4 *
 * sparse_count an fp32 per-key dI buffer [batch*s1, s2] (at most 512 MiB; the key-major
 * d_key_index pass), the row losses and the teacher's token lists. Needs no
 * initialisation. No counterpart in the reference (it allocates its buffers per call,
 * sparse_lightning_indexer_grad_kl_loss_triton.py:375-392).
 */
size_t dsa_sli_grad_workspace_bytes(int batch, int s1, int s2, int sparse_count, int d_idx);

/*
 * Sparse lightning-indexer grad KL loss, BSND, sparse_mode 3 (replaces
 * _sparse_lightning_indexer_grad_kl_loss_core,
 * sparse_lightning_indexer_grad_kl_loss_triton.py:333-440; semantics of
 * sli_grad_kl_loss_numpy.py:17-180 with the row bounds of the reference kernel
 * :63-69). Per query row (b, s1 < act_q[b]) the first
 * n = min(sparse_count, max(act_k[b] - act_q[b] + s1 + 1, 0)) ids of
 * sparse_indices[b, s1, 0, :], each clipped to [0, s2 - 1]:
 *   p[k]  = (1/N1) sum_h exp(score[h,k] - sm_max) / (sm_sum + 1e-8),
 *           score = (q . k + q_rope . k_rope) * scale
 *   I[k]  = sum_g w[g] relu(qi[g] . ki[k]),  sI = softmax(I) (1e-8 in the sum)
 *   loss  = sum over rows and k of max(p,1e-8) (log max(p,1e-8) - log max(sI,1e-8))
 *   d_weights[g] = sum_k relu[g,k] (sI - p)[k];  ds[g,k] = (sI - p)[k] w[g] [relu > 0]
 *   d_query_index[g] = sum_k ds[g,k] ki[k];  d_key_index[id_k] += sum_g ds[g,k] qi[g]
 * query [B,S1,N1,D], key [B,S2,1,D], query_rope / key_rope [..,64] (both NULL with
 * dr = 0), query_index [B,S1,Nidx1,D_idx], key_index [B,S2,1,D_idx] (io dtype),
 * weights [B,S1,Nidx1] (w_dtype), sm_max / sm_sum [B,1,S1,N1] fp32 (the forward's
 * stats), act_q / act_k [B]. Outputs in the inputs' dtypes; loss: one fp32.
 * D in {128,256,512}, D_idx in {128,256,512}, N1 <= 128, Nidx1 <= 128, sparse_count <= 2048.
 */
int dsa_sli_grad_kl_loss(const void* query, const void* key, const void* query_rope, const void* key_rope,
                         const void* query_index, const void* key_index, const void* weights, int io_dtype,
                         int w_dtype, const int32_t* sparse_indices, int sparse_count, const float* sm_max,
                         const float* sm_sum, const int32_t* act_q, const int32_t* act_k, int batch, int s1,
                         int s2, int n1, int d, int dr, int nidx1, int d_idx, float scale,
                         void* d_query_index, void* d_key_index, void* d_weights, float* loss,
                         void* workspace, size_t workspace_bytes, void* stream);

/*
 * Dense lightning-indexer softmax LSE, BSND, sparse_mode 3 (replaces
 * _dense_index_stats_core, dense_loss_backward_triton.py:354-378, behind
 * npu_dense_lightning_indexer_softmax_lse_triton :776-806). Per query row
 * (b, s1 < act_q[b]) over keys t < min(max(act_k[b] - act_q[b] + s1 + 1, 0), s2):
 * softmax_max_index = max_t I[t], softmax_sum_index = sum_t exp(I[t] - max),
 * I[t] = sum_g w[g] relu(qi[g] . ki[t]); other rows get (-inf, 0). Outputs [B*S1] fp32
 * (the reference's [B,1,S1]). D_idx in {128,256,512}, Nidx1 <= 128, any s2. Needs no
 * workspace.
 */
int dsa_dense_li_softmax_lse(const void* query_index, const void* key_index, const void* weights, int io_dtype,
                             int w_dtype, const int32_t* act_q, const int32_t* act_k, int batch, int s1, int s2,
                             int nidx1, int d_idx, float* softmax_max_index, float* softmax_sum_index,
                             void* stream);

/* Workspace bytes for dsa_dense_li_grad_kl_loss (the sparse loss's layout with s2 slots
 * per row); no initialisation needed. No counterpart in the reference (it allocates
 * per call, dense_loss_backward_triton.py:393-605). */
size_t dsa_dense_li_grad_workspace_bytes(int batch, int s1, int s2, int d_idx);

/*
 * Dense lightning-indexer grad KL loss, BSND, sparse_mode 3 (replaces
 * _dense_loss_backward_core / _dense_loss_backward_with_index_core,
 * dense_loss_backward_triton.py:393-605, behind dense_loss_backward_triton :709-774).
 * dsa_sli_grad_kl_loss with every visible key t < min(max(act_k - act_q + s1 + 1, 0), s2)
 * as a slot, and:
 *  - teacher over grouped key heads: key / key_rope [B,S2,N2,D(+64)], head h reads key
 *    head h / G (G = N1 / N2) and sm_max / sm_sum [B,N2,S1,G] at (b, h / G, s1, h % G);
 *  - indexer softmax sI = exp(I - max_index) / max(sum_index, 1e-8) from the given stats
 *    (max_index / sum_index [B*S1] fp32; a row with sum_index <= 0 gets zero gradients
 *    and no loss), or, with both NULL, from the row's own max and sum.
 * D in {128,256,512}, D_idx in {128,256,512}, N1 <= 128, Nidx1 <= 128, any s2.
 */
int dsa_dense_li_grad_kl_loss(const void* query, const void* key, const void* query_rope, const void* key_rope,
                              const void* query_index, const void* key_index, const void* weights, int io_dtype,
                              int w_dtype, const float* sm_max, const float* sm_sum, const float* max_index,
                              const float* sum_index, const int32_t* act_q, const int32_t* act_k, int batch,
                              int s1, int s2, int n1, int n2, int d, int dr, int nidx1, int d_idx, float scale,
                              void* d_query_index, void* d_key_index, void* d_weights, float* loss,
                              void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DSA_MI355X_H */
