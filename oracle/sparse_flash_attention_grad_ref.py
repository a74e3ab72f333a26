"""numpy restatement of the sparse_flash_attention_grad golden (test infrastructure only).

Semantics follow sparse_flash_attention_grad_numpy.py:34-143 (MLA-absorb, N2 = 1):

* the row selection and gathered token positions are the forward's
  (``gather_positions``, sparse_flash_attention_numpy.py:38-60; mode-3 rows with
  ``s1 < aq - ak`` and rows with ``threshold <= 0`` or no token contribute nothing);
* per row and head, with the forward's stats: ``P = exp(score - sm_max) / sm_sum``
  where ``score = (q_nope . k_nope + q_rope . k_rope) * scale`` (grad_numpy:117-120),
  ``dP = dO . k_nope`` (value aliases the key), ``delta = dO . O`` (O the forward
  output), ``dS = P * (dP - delta) * scale`` (grad_numpy:121-123);
* ``d_query = dS @ k_nope``, ``d_query_rope = dS @ k_rope`` per row; ``d_key``,
  ``d_key_rope`` (from ``dS^T q``) and ``d_value`` (from ``P^T dO``) are scatter-added
  over the gathered positions, a position selected by several rows summing all of
  them (grad_numpy:125-134, ``np.add.at``);
* the five outputs are rounded to the io dtype at the end (grad_numpy:136-143).

Everything is fp32, as in the golden. ``sparse_flash_attention_grad`` mirrors the
host wrapper sparse_flash_attention_grad_triton.py:498-677: TND inputs are de-packed
with the cumulative lengths, the stats ``(1, T1, N1)`` become ``(B, 1, S1, N1)``,
and the outputs are re-packed.
"""
import numpy as np

from .lightning_indexer_ref import tnd_cumsum_to_per_batch, tnd_to_bsnd, bsnd_to_tnd
from .sparse_flash_attention_ref import gather_positions, _round_io


def sfa_grad_golden_bsnd(q_nope, k_nope, sparse_indices, d_out, out, softmax_max, softmax_sum,
                         q_rope, k_rope, scale_value, act_q, act_k, sparse_block_size=1,
                         sparse_mode=3, io_dtype="bf16"):
    """BSND golden (sparse_flash_attention_grad_numpy.py:34-143). The heads of a row are
    evaluated together; every head's terms are the golden's per-head expressions.
    Returns (d_query, d_key, d_value, d_query_rope, d_key_rope), fp32 rounded to io dtype."""
    f = lambda x: np.asarray(x, np.float32)
    qn, kn, qr, kr, do, o = f(q_nope), f(k_nope), f(q_rope), f(k_rope), f(d_out), f(out)
    smax, ssum = f(softmax_max), f(softmax_sum)
    B, S1, N1, D = qn.shape
    S2, Dr = kn.shape[1], qr.shape[-1]
    scale = np.float32(scale_value)
    dq = np.zeros((B, S1, N1, D), np.float32)
    dqr = np.zeros((B, S1, N1, Dr), np.float32)
    dk = np.zeros((B, S2, 1, D), np.float32)
    dkr = np.zeros((B, S2, 1, Dr), np.float32)
    dv = np.zeros((B, S2, 1, D), np.float32)
    for b in range(B):
        aq, ak = int(act_q[b]), int(act_k[b])
        for s1 in range(aq):
            if sparse_mode != 0 and s1 < aq - ak:
                continue
            threshold = ak if sparse_mode == 0 else ak - aq + s1 + 1
            if threshold <= 0:
                continue
            pos = gather_positions(sparse_indices[b, s1, 0, :], sparse_block_size, threshold, ak)
            if not pos:
                continue
            pos = np.asarray(pos, np.int64)
            kn_sp, kr_sp = kn[b, pos, 0, :], kr[b, pos, 0, :]                  # [P, D], [P, Dr]
            scores = (qn[b, s1] @ kn_sp.T + qr[b, s1] @ kr_sp.T) * scale       # [N1, P]
            p = np.exp(scores - smax[b, 0, s1][:, None]) / ssum[b, 0, s1][:, None]
            dp = do[b, s1] @ kn_sp.T                                           # [N1, P]
            delta = np.sum(do[b, s1] * o[b, s1], axis=1)                       # [N1]
            ds = p * (dp - delta[:, None]) * scale                             # [N1, P]
            dq[b, s1] += ds @ kn_sp
            dqr[b, s1] += ds @ kr_sp
            if len(np.unique(pos)) == len(pos):   # distinct positions: a plain indexed add is the same sum
                dk[b, pos, 0, :] += ds.T @ qn[b, s1]
                dkr[b, pos, 0, :] += ds.T @ qr[b, s1]
                dv[b, pos, 0, :] += p.T @ do[b, s1]
            else:
                np.add.at(dk[b, :, 0, :], pos, ds.T @ qn[b, s1])
                np.add.at(dkr[b, :, 0, :], pos, ds.T @ qr[b, s1])
                np.add.at(dv[b, :, 0, :], pos, p.T @ do[b, s1])
    r = lambda x: _round_io(x, io_dtype)
    return r(dq), r(dk), r(dv), r(dqr), r(dkr)


def sparse_flash_attention_grad(query, key, value, sparse_indices, d_out, out, softmax_max,
                                softmax_sum, scale_value=1.0, query_rope=None, key_rope=None,
                                actual_seq_lengths_query=None, actual_seq_lengths_kv=None,
                                sparse_block_size=1, layout="BSND", sparse_mode=3, io_dtype="bf16"):
    """Oracle twin of ``sparse_flash_attention_grad_triton`` (sparse_flash_attention_grad_triton.py:
    498-677) on numpy arrays; ``value`` is ignored (MLA-absorb). Returns
    (d_query, d_key, d_value, d_query_rope, d_key_rope) in the inputs' layouts."""
    f = lambda x: np.asarray(x, np.float32)
    si = np.asarray(sparse_indices, np.int32)
    if layout == "TND":
        act_q = tnd_cumsum_to_per_batch(actual_seq_lengths_query)
        act_k = tnd_cumsum_to_per_batch(actual_seq_lengths_kv)
        q, qr, do, o = (tnd_to_bsnd(f(x), act_q) for x in (query, query_rope, d_out, out))
        si = tnd_to_bsnd(si, act_q)
        k, kr = tnd_to_bsnd(f(key), act_k), tnd_to_bsnd(f(key_rope), act_k)
        # (1, T1, N1) -> (T1, 1, N1) -> (B, S1, 1, N1) -> (B, 1, S1, N1)
        smax = tnd_to_bsnd(f(softmax_max).transpose(1, 0, 2), act_q).transpose(0, 2, 1, 3)
        ssum = tnd_to_bsnd(f(softmax_sum).transpose(1, 0, 2), act_q).transpose(0, 2, 1, 3)
    else:
        q, qr, do, o, k, kr = (f(x) for x in (query, query_rope, d_out, out, key, key_rope))
        smax, ssum = f(softmax_max), f(softmax_sum)
        B, S1, S2 = q.shape[0], q.shape[1], k.shape[1]
        act_q = np.full(B, S1, np.int32) if actual_seq_lengths_query is None else np.asarray(actual_seq_lengths_query, np.int32)
        act_k = np.full(B, S2, np.int32) if actual_seq_lengths_kv is None else np.asarray(actual_seq_lengths_kv, np.int32)
    dq, dk, dv, dqr, dkr = sfa_grad_golden_bsnd(q, k, si, do, o, smax, ssum, qr, kr, scale_value,
                                                act_q, act_k, sparse_block_size, sparse_mode, io_dtype)
    if layout == "TND":
        dq, dqr = bsnd_to_tnd(dq, act_q), bsnd_to_tnd(dqr, act_q)
        dk, dkr, dv = bsnd_to_tnd(dk, act_k), bsnd_to_tnd(dkr, act_k), bsnd_to_tnd(dv, act_k)
    return dq, dk, dv, dqr, dkr
