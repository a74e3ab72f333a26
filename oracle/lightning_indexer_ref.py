"""numpy restatement of the lightning_indexer golden (test infrastructure only).

Semantics follow lightning_indexer_numpy.py:38-111 (``lightning_indexer_golden_bsnd``):

* per (b, s1 < act_q[b], n2):
  ``score[s2] = sum_{g in group(n2)} relu(q[b,s1,g,:] . k[b,s2,n2,:]) * w[b,s1,g]``
  accumulated in fp32, g in ascending order (numpy_golden:75-83);
* sparse_mode 3: ``s2 >= min(max(act_k - act_q + s1 + 1, 0), S2)`` and
  ``s2 >= act_k`` are -inf; sparse_mode 0: only ``s2 >= act_k`` (numpy_golden:85-90);
* scores are quantised to the value dtype (bf16 RNE / fp16) BEFORE ordering
  (numpy_golden:92);
* order: score descending, ties by ascending index (lexsort, numpy_golden:94-97);
* the first ``min(act_k, sparse_count)`` sorted entries are emitted, -inf ones
  are skipped leaving index -1 and value 0 (numpy_golden:99-105); rows with
  ``s1 >= act_q`` stay all -1 / 0.

The TND entry mirrors lightning_indexer_triton.py:294-340 and :504-552:
cumulative actual_seq_lengths are differenced into per-batch lengths, the
packed rows are zero-padded into BSND, the BSND golden runs, and the rows are
packed back.
"""
import numpy as np

from .numerics import quantize


def _row_scores(q_row, k_bn, w_row, g0, G):
    """fp32 scores of one (b, s1, n2) row before masking (numpy_golden:75-83).

    q_row [N1, D], k_bn [S2, D] (key head n2), w_row [N1]."""
    dots = k_bn @ q_row[g0:g0 + G].T            # [S2, G], fp32 BLAS like the golden's k_vec @ q_vec
    scores = np.zeros(k_bn.shape[0], dtype=np.float32)
    for g in range(G):                           # same g order as the golden
        scores += np.maximum(dots[:, g], np.float32(0.0)) * w_row[g0 + g]
    return scores


def visible_len(s1, act_q, act_k, S2, sparse_mode):
    """Number of visible keys (a prefix) for a row (numpy_golden:85-90)."""
    if sparse_mode == 3:
        return max(0, min(min(max(act_k - act_q + s1 + 1, 0), S2), act_k))
    return max(0, min(act_k, S2))


def li_row_scores(q, k, w, b, s1, n2, act_q, act_k, sparse_mode=3):
    """Masked fp32 score row (before quantisation) for one (b, s1, n2)."""
    B, S1, N1, D = q.shape
    S2, N2 = k.shape[1], k.shape[2]
    G = N1 // N2
    s = _row_scores(q[b, s1].astype(np.float32), k[b, :, n2, :].astype(np.float32),
                    w[b, s1].astype(np.float32), n2 * G, G)
    L = visible_len(s1, int(act_q[b]), int(act_k[b]), S2, sparse_mode)
    s[L:] = -np.inf
    return s


def li_row_scores_f64(q, k, w, b, s1, n2, act_q, act_k, sparse_mode=3):
    """Same row in float64 (the 'true' value used to bound rounding ambiguity)."""
    B, S1, N1, D = q.shape
    S2, N2 = k.shape[1], k.shape[2]
    G = N1 // N2
    dots = k[b, :, n2, :].astype(np.float64) @ q[b, s1, n2 * G:(n2 + 1) * G].astype(np.float64).T
    s = (np.maximum(dots, 0.0) * w[b, s1, n2 * G:(n2 + 1) * G].astype(np.float64)).sum(axis=1)
    L = visible_len(s1, int(act_q[b]), int(act_k[b]), S2, sparse_mode)
    s[L:] = -np.inf
    return s


def select_topk(scores_q, act_k, sparse_count):
    """Stable top-k of one quantised row (numpy_golden:94-105).

    Returns (indices int32 [sparse_count], values fp32 [sparse_count])."""
    S2 = scores_q.shape[0]
    idx_out = np.full(sparse_count, -1, dtype=np.int32)
    val_out = np.zeros(sparse_count, dtype=np.float32)
    indices = np.arange(S2, dtype=np.int32)
    order = np.lexsort((indices.astype(np.float32), -scores_q))
    n = min(int(act_k), sparse_count, S2)
    sel = indices[order[:n]]
    ok = scores_q[sel] != -np.inf
    # -inf entries sort last, so the valid ones form a prefix of the slots
    nv = int(ok.sum())
    idx_out[:nv] = sel[:nv]
    val_out[:nv] = scores_q[sel[:nv]]
    return idx_out, val_out


def li_golden_bsnd(q, k, w, act_q, act_k, sparse_count=2048, sparse_mode=3,
                   return_value=False, value_dtype="bf16", rows=None):
    """BSND golden (lightning_indexer_numpy.py:38-111).

    q [B,S1,N1,D], k [B,S2,N2,D], w [B,S1,N1] (any float dtype, values taken as fp32).
    ``rows``: optional iterable of (b, s1) to evaluate (the others stay -1 / 0);
    used for stride-sampled checks and the CPU baseline at large shapes.
    Returns (indices [B,S1,N2,k] int32, values [B,S1,N2,k] fp32)."""
    q = np.asarray(q, dtype=np.float32)
    k = np.asarray(k, dtype=np.float32)
    w = np.asarray(w, dtype=np.float32)
    B, S1, N1, D = q.shape
    _, S2, N2, _ = k.shape
    G = N1 // N2
    idx = np.full((B, S1, N2, sparse_count), -1, dtype=np.int32)
    val = np.zeros((B, S1, N2, sparse_count), dtype=np.float32)
    if rows is None:
        rows = [(b, s1) for b in range(B) for s1 in range(min(int(act_q[b]), S1))]
    for b, s1 in rows:
        if s1 >= int(act_q[b]) or s1 >= S1:
            continue
        for n2 in range(N2):
            s = _row_scores(q[b, s1], k[b, :, n2, :], w[b, s1], n2 * G, G)
            L = visible_len(s1, int(act_q[b]), int(act_k[b]), S2, sparse_mode)
            s[L:] = -np.inf
            sq = quantize(s, value_dtype)
            idx[b, s1, n2], val[b, s1, n2] = select_topk(sq, int(act_k[b]), sparse_count)
    if not return_value:
        val = np.zeros_like(val)
    return idx, val


# ---------------------------------------------------------------- layouts
def tnd_cumsum_to_per_batch(cu):
    """lightning_indexer_triton.py:294-296: cumulative lengths -> per-batch lengths."""
    cu = np.asarray(cu, dtype=np.int64)
    return np.diff(np.concatenate([[0], cu])).astype(np.int32)


def tnd_to_bsnd(t, lens):
    """lightning_indexer_triton.py:299-320: [T,...] -> zero-padded [B,maxS,...]."""
    lens = [int(x) for x in lens]
    maxs = max(lens) if lens else 0
    out = np.zeros((len(lens), maxs) + tuple(t.shape[1:]), dtype=t.dtype)
    start = 0
    for b, L in enumerate(lens):
        if L > 0:
            out[b, :L] = t[start:start + L]
            start += L
    return out


def bsnd_to_tnd(t, lens):
    """lightning_indexer_triton.py:323-340: [B,S,...] -> packed [T,...]."""
    lens = [int(x) for x in lens]
    parts = [t[b, :L] for b, L in enumerate(lens) if L > 0]
    if not parts:
        return np.zeros((0,) + tuple(t.shape[2:]), dtype=t.dtype)
    return np.concatenate(parts, axis=0)


def lightning_indexer(query, key, weights, actual_seq_lengths_query=None,
                      actual_seq_lengths_key=None, block_table=None, layout_query="BSND",
                      layout_key="BSND", sparse_count=2048, sparse_mode=3,
                      return_value=False, value_dtype="bf16", rows=None):
    """Oracle twin of ``lightning_indexer_triton`` (lightning_indexer_triton.py:466-554)
    on numpy arrays. ``value_dtype`` is the query dtype ("bf16" / "fp16").

    ``layout_key="PA_BSND"`` (no counterpart in the reference, which rejects a block
    table, :501-502): the paged key cache is de-paged the way the reference de-pages
    the SFA cache (``pa_to_bsnd``, sparse_flash_attention_triton.py:1012-1033: a -1
    block is a zero key row) and the kv lengths are per batch; then the BSND golden."""
    is_pa = layout_key == "PA_BSND"
    if block_table is not None and not is_pa:
        raise ValueError("PA_BSND / block_table not supported in lightning_indexer")
    is_tnd = layout_query == "TND"
    if is_pa:
        from .sparse_flash_attention_ref import pa_to_bsnd
        bt = np.asarray(block_table)
        k = pa_to_bsnd(np.asarray(key, np.float32), bt, bt.shape[1] * key.shape[1])
        B = bt.shape[0]
        act_k = (np.full(B, k.shape[1], np.int32) if actual_seq_lengths_key is None
                 else np.asarray(actual_seq_lengths_key, np.int32))
    if is_tnd:
        act_q = tnd_cumsum_to_per_batch(actual_seq_lengths_query)
        q = tnd_to_bsnd(np.asarray(query, np.float32), act_q)
        w = tnd_to_bsnd(np.asarray(weights, np.float32), act_q)
        if not is_pa:
            act_k = tnd_cumsum_to_per_batch(actual_seq_lengths_key)
            k = tnd_to_bsnd(np.asarray(key, np.float32), act_k) if layout_key == "TND" else np.asarray(key, np.float32)
    elif is_pa:
        q, w = np.asarray(query, np.float32), np.asarray(weights, np.float32)
        act_q = np.full(q.shape[0], q.shape[1], np.int32) if actual_seq_lengths_query is None else np.asarray(actual_seq_lengths_query, np.int32)
    else:
        q, k, w = (np.asarray(x, np.float32) for x in (query, key, weights))
        B = q.shape[0]
        act_q = np.full(B, q.shape[1], np.int32) if actual_seq_lengths_query is None else np.asarray(actual_seq_lengths_query, np.int32)
        act_k = np.full(B, k.shape[1], np.int32) if actual_seq_lengths_key is None else np.asarray(actual_seq_lengths_key, np.int32)
    N1, N2 = q.shape[2], k.shape[2]
    if N1 % N2 != 0:
        raise ValueError(f"N1({N1}) must be divisible by N2({N2})")
    idx, val = li_golden_bsnd(q, k, w, act_q, act_k, sparse_count, sparse_mode,
                              return_value=return_value, value_dtype=value_dtype, rows=rows)
    if is_tnd:
        idx, val = bsnd_to_tnd(idx, act_q), bsnd_to_tnd(val, act_q)
    return idx, val
