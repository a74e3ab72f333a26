"""numpy restatement of the dense lightning-indexer loss goldens (test
infrastructure only): the dense warm-up stage of the indexer's training.

* ``dense_softmax_lse`` <- test_dense_loss_backward_triton.py:124-159
  (``_dense_indexer_lse_numpy``): per query row (b, s1 < act_q) over the visible
  keys ``t < min(max(act_k - act_q + s1 + 1, 0), act_k, S2)``, the max and the sum of
  ``exp(I - max)`` of ``I[t] = sum_g w[g] relu(qi[g] . ki[t])``; other rows keep
  ``(-inf, 0)``. Shapes (B, 1, S1) fp32.
* ``dense_loss_backward`` <- test_dense_loss_backward_triton.py:230-315
  (``_dense_loss_backward_numpy``): the sparse KL loss over every visible key
  ``t < min(max(act_k - act_q + s1 + 1, 0), S2)`` with the indexer softmax normalised
  by the given stats (``sI = exp(I - max_index) / max(sum_index, 1e-8)``, rows with
  ``sum_index <= 0`` skipped) and the teacher from grouped attention heads: head h
  reads key head ``h // G`` and its stats ``softmax_max[b, h // G, s1, h % G]``
  (``[B, N2, S1, G]``).
"""
import numpy as np

from .sparse_flash_attention_ref import _round_io

EPS = 1e-8


def dense_softmax_lse(qi, ki, w, act_q=None, act_k=None):
    qi, ki, w = (np.asarray(x, np.float32) for x in (qi, ki, w))
    B, S1, G, Di = qi.shape
    S2 = ki.shape[1]
    act_q = np.full(B, S1) if act_q is None else np.asarray(act_q)
    act_k = np.full(B, S2) if act_k is None else np.asarray(act_k)
    mx = np.full((B, 1, S1), -np.inf, np.float32)
    sm = np.zeros((B, 1, S1), np.float32)
    for b in range(B):
        aq, ak = int(act_q[b]), int(act_k[b])
        for s1 in range(min(S1, aq)):
            n = min(max(ak - aq + s1 + 1, 0), ak, S2)
            if n <= 0:
                continue
            ii = (w[b, s1, :, None] * np.maximum(qi[b, s1] @ ki[b, :n, 0].T, 0.0)).sum(0)
            m = np.float32(ii.max())
            mx[b, 0, s1] = m
            sm[b, 0, s1] = np.float32(np.exp(ii - m).sum())
    return mx, sm


def dense_loss_backward(q, k, qr, kr, qi, ki, w, sm_max, sm_sum, max_index, sum_index, scale,
                        act_q=None, act_k=None, io_dtype="fp16", w_dtype=None):
    f = lambda x: np.asarray(x, np.float32)
    q, k, qi, ki, w, sm_max, sm_sum = (f(x) for x in (q, k, qi, ki, w, sm_max, sm_sum))
    qr = None if qr is None else f(qr)
    kr = None if kr is None else f(kr)
    mxi, smi = f(max_index).reshape(-1), f(sum_index).reshape(-1)
    B, S1, N1, D = q.shape
    S2, N2 = k.shape[1], k.shape[2]
    Gq = N1 // N2
    G, Di = qi.shape[2], qi.shape[3]
    act_q = np.full(B, S1) if act_q is None else np.asarray(act_q)
    act_k = np.full(B, S2) if act_k is None else np.asarray(act_k)
    dqi = np.zeros_like(qi)
    dki = np.zeros((B, S2, 1, Di), np.float32)
    dw = np.zeros((B, S1, G), np.float32)
    loss = 0.0
    heads = np.arange(N1)
    kvh, gh = heads // Gq, heads % Gq
    for b in range(B):
        aq, ak = int(act_q[b]), int(act_k[b])
        for s1 in range(min(S1, aq)):
            n = min(max(ak - aq + s1 + 1, 0), S2)
            i_sum = float(smi[b * S1 + s1])
            if n <= 0 or i_sum <= 0.0:
                continue
            kiv = ki[b, :n, 0, :]
            relu = np.maximum(qi[b, s1] @ kiv.T, 0.0)                                   # [G, n]
            ii = (w[b, s1, :, None] * relu).sum(0)
            student = np.exp(ii - float(mxi[b * S1 + s1])) / max(i_sum, EPS)
            # head h against key head kvh[h] (no gather copy when every head has its own key head)
            kh = (lambda x: x if Gq == 1 else x[:, kvh, :])
            sc = np.einsum("hd,nhd->hn", q[b, s1], kh(k[b, :n]))                          # [N1, n]
            if qr is not None:
                sc = sc + np.einsum("hd,nhd->hn", qr[b, s1], kh(kr[b, :n]))
            sc = sc * np.float32(scale)
            m = sm_max[b, kvh, s1, gh][:, None]
            l = sm_sum[b, kvh, s1, gh][:, None]
            p = (np.exp(sc - m) / (l + EPS)).sum(0) * np.float32(1.0 / N1)
            di = student - p
            ps, qs = np.maximum(p, EPS), np.maximum(student, EPS)
            loss += float(np.sum(ps * (np.log(ps) - np.log(qs))))
            dw[b, s1] = relu @ di
            ds = (di[None, :] * w[b, s1][:, None]) * (relu > 0)
            dqi[b, s1] = ds @ kiv
            dki[b, :n, 0] += ds.T @ qi[b, s1]
    return (_round_io(dqi, io_dtype), _round_io(dki, io_dtype), _round_io(dw, w_dtype or io_dtype),
            np.array([loss], np.float32))
