"""numpy restatement of the sparse_flash_attention golden (test infrastructure only).

Semantics follow sparse_flash_attention_numpy.py:38-160:

* ``gather_positions`` (numpy_golden:38-60): only the first
  ``min(count, ceil(threshold / bs))`` block ids are scanned, the scan STOPS at
  the first -1, each id expands to tokens ``[id*bs, min(id*bs+bs, act_k))``
  clipped to ``threshold``; ids starting at or beyond ``threshold`` are skipped.
* per (b, s1 < act_q): sparse_mode 3 skips rows with ``s1 < aq - ak``
  (numpy_golden:125-126); ``threshold = ak`` (mode 0) or ``ak - aq + s1 + 1``
  (mode 3); ``threshold <= 0`` or no gathered token skips the row (output 0,
  sm_max = sm_sum = 0).
* ``score = (q_nope . k_nope + q_rope . k_rope) * scale`` (fp32),
  ``probs = round(exp(score - max) / sum)`` to the io dtype, ``out = probs @ k_nope``
  (value aliases key, MLA-absorb), then ``out`` rounded to the io dtype;
  ``sm_max = max``, ``sm_sum = sum(exp(score - max))`` (numpy_golden:143-159).

Layouts mirror sparse_flash_attention_triton.py:1353-1450: TND q/kv are
de-packed with cumulative lengths, PA_BSND kv is de-paged through the block
table (``_pa_to_bsnd``, :1012-1033) with per-batch (not cumulative) kv lengths,
TND outputs are re-packed and the softmax stats become ``(1, T1, N1)``.
"""
import math

import numpy as np

from .numerics import round_bf16, round_fp16
from .lightning_indexer_ref import tnd_cumsum_to_per_batch, tnd_to_bsnd, bsnd_to_tnd


def gather_positions(sparse_idx_row, sparse_block_size, threshold, act_k):
    """sparse_flash_attention_numpy.py:38-60 (CANN gatherKV contract)."""
    count = sparse_idx_row.shape[0]
    valid_count = min(count, math.ceil(threshold / sparse_block_size))
    pos = []
    for i in range(valid_count):
        sid = int(sparse_idx_row[i])
        if sid == -1:
            break
        begin = sid * sparse_block_size
        end = min(begin + sparse_block_size, act_k)
        if begin >= threshold:
            continue
        pos.extend(range(begin, min(end, threshold)))
    return pos


def _round_io(x, io_dtype):
    if io_dtype == "fp16":
        return round_fp16(x)
    if io_dtype == "bf16":
        return round_bf16(x)
    return np.asarray(x, np.float32)


def sfa_golden_bsnd(q_nope, k_nope, sparse_indices, q_rope, k_rope, scale_value, act_q, act_k,
                    sparse_block_size=1, sparse_mode=3, io_dtype="bf16", rows=None):
    """BSND golden (sparse_flash_attention_numpy.py:63-160).

    Heads of one query row are evaluated together (``q_full[N1, D+Dr] @ k_sp.T``);
    each head's softmax is independent, exactly as the golden's per-head loop.
    ``rows``: optional iterable of (b, s1) to evaluate (others stay 0).
    Returns (out [B,S1,N1,D] fp32 rounded to io dtype, sm_max, sm_sum [B,1,S1,N1])."""
    qn = np.asarray(q_nope, np.float32)
    kn = np.asarray(k_nope, np.float32)
    qr = np.asarray(q_rope, np.float32)
    kr = np.asarray(k_rope, np.float32)
    B, S1, N1, D = qn.shape
    out = np.zeros((B, S1, N1, D), np.float32)
    smax = np.zeros((B, 1, S1, N1), np.float32)
    ssum = np.zeros((B, 1, S1, N1), np.float32)
    if rows is None:
        rows = [(b, s1) for b in range(B) for s1 in range(int(act_q[b]))]
    for b, s1 in rows:
        aq, ak = int(act_q[b]), int(act_k[b])
        if s1 >= aq:
            continue
        if sparse_mode != 0 and s1 < aq - ak:
            continue
        threshold = ak if sparse_mode == 0 else ak - aq + s1 + 1
        if threshold <= 0:
            continue
        pos = gather_positions(sparse_indices[b, s1, 0, :], sparse_block_size, threshold, ak)
        if not pos:
            continue
        pos = np.asarray(pos, np.int64)
        k_sp = np.concatenate([kn[b, pos, 0, :], kr[b, pos, 0, :]], axis=-1)   # [P, D+Dr]
        v_sp = kn[b, pos, 0, :]                                               # [P, D]
        q_full = np.concatenate([qn[b, s1], qr[b, s1]], axis=-1)             # [N1, D+Dr]
        scores = (q_full @ k_sp.T) * np.float32(scale_value)                  # [N1, P]
        m = scores.max(axis=1, keepdims=True)
        e = np.exp(scores - m)
        ssum_row = e.sum(axis=1, keepdims=True)
        probs = _round_io(e / ssum_row, io_dtype)
        out[b, s1] = probs @ v_sp
        smax[b, 0, s1] = m[:, 0]
        ssum[b, 0, s1] = ssum_row[:, 0]
    out = _round_io(out, io_dtype)
    return out, smax, ssum


def pa_to_bsnd(cache, block_table, max_s2):
    """sparse_flash_attention_triton.py:1012-1033: de-page [nblk,bs,N,Dx] -> [B,max_s2,N,Dx]."""
    nblk, bs, N, Dx = cache.shape
    B, mb = block_table.shape
    out = np.zeros((B, max_s2, N, Dx), dtype=cache.dtype)
    for b in range(B):
        for i in range(mb):
            blk = int(block_table[b, i])
            if blk == -1:
                continue
            dst = i * bs
            if dst >= max_s2:
                break
            end = min(dst + bs, max_s2)
            out[b, dst:end] = cache[blk, :end - dst]
    return out


def sparse_flash_attention(query, key, value, sparse_indices, scale_value=1.0, block_table=None,
                           actual_seq_lengths_query=None, actual_seq_lengths_kv=None,
                           query_rope=None, key_rope=None, sparse_block_size=1,
                           layout_query="BSND", layout_kv="BSND", sparse_mode=0,
                           return_softmax_lse=False, block_size=0, io_dtype="bf16", rows=None):
    """Oracle twin of ``sparse_flash_attention_triton`` (sparse_flash_attention_triton.py:1295-1455)
    on numpy arrays. ``value`` is ignored (MLA-absorb). Returns (out, sm_max, sm_sum) with the
    reference's output layouts; the stats are zeros when ``return_softmax_lse`` is False."""
    is_tnd_q = layout_query == "TND"
    is_tnd_kv = layout_kv == "TND"
    is_pa = layout_kv == "PA_BSND"
    f = lambda x: np.asarray(x, np.float32)
    if is_tnd_q:
        act_q = tnd_cumsum_to_per_batch(actual_seq_lengths_query)
        q = tnd_to_bsnd(f(query), act_q)
        qr = tnd_to_bsnd(f(query_rope), act_q)
        si = tnd_to_bsnd(np.asarray(sparse_indices, np.int32), act_q)
    else:
        q, qr, si = f(query), f(query_rope), np.asarray(sparse_indices, np.int32)
        B = q.shape[0]
        act_q = np.full(B, q.shape[1], np.int32) if actual_seq_lengths_query is None else np.asarray(actual_seq_lengths_query, np.int32)
    if is_tnd_kv:
        act_k = tnd_cumsum_to_per_batch(actual_seq_lengths_kv)
        k = tnd_to_bsnd(f(key), act_k)
        kr = tnd_to_bsnd(f(key_rope), act_k)
    elif is_pa:
        bs = block_size or key.shape[1]
        max_s2 = block_table.shape[1] * bs
        k = pa_to_bsnd(f(key), np.asarray(block_table), max_s2)
        kr = pa_to_bsnd(f(key_rope), np.asarray(block_table), max_s2)
        act_k = np.asarray(actual_seq_lengths_kv, np.int32)
    else:
        k, kr = f(key), f(key_rope)
        act_k = np.full(q.shape[0], k.shape[1], np.int32) if actual_seq_lengths_kv is None else np.asarray(actual_seq_lengths_kv, np.int32)
    out, smax, ssum = sfa_golden_bsnd(q, k, si, qr, kr, scale_value, act_q, act_k,
                                      sparse_block_size, sparse_mode, io_dtype, rows=rows)
    if not return_softmax_lse:
        smax = np.zeros_like(smax)
        ssum = np.zeros_like(ssum)
    if is_tnd_q:
        out = bsnd_to_tnd(out, act_q)
        smax = bsnd_to_tnd(smax.transpose(0, 2, 1, 3), act_q).transpose(1, 0, 2)
        ssum = bsnd_to_tnd(ssum.transpose(0, 2, 1, 3), act_q).transpose(1, 0, 2)
    return out, smax, ssum
