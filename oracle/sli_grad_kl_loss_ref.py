"""numpy restatement of the sparse lightning-indexer grad KL-loss golden (test
infrastructure only).

Semantics follow sli_grad_kl_loss_numpy.py:17-180 (``numpy_reference``) with the
row bounds of the Triton kernel (sparse_lightning_indexer_grad_kl_loss_triton.py:
63-69), which reduce to the golden's when the actual lengths are the shapes:

* per query row (b, s1 < act_q): ``n = min(topK, max(act_k - act_q + s1 + 1, 0))``
  slots of ``sparse_indices[b, s1, 0, :]`` are used, each clipped to ``[0, S2-1]``
  (no -1 semantics; repeated ids count once per slot);
* teacher ``p[k] = (1/N1) sum_h exp(score[h,k] - sm_max[h]) / (sm_sum[h] + 1e-8)``,
  ``score = (q . k + q_rope . k_rope) * scale`` (golden :82-95);
* student ``I[k] = sum_g w[g] relu(qi[g] . ki[k])`` (:67-79),
  ``sI = exp(I - max I) / (sum exp(I - max I) + 1e-8)`` (:99-107);
* ``dI = sI - p``, ``loss = sum max(p, 1e-8) (log max(p, 1e-8) - log max(sI, 1e-8))``
  over all rows (:110-120);
* ``dW[g] = sum_k relu[g,k] dI[k]``, ``ds[g,k] = dI[k] w[g] [relu > 0]``,
  ``dQI[g] = sum_k ds[g,k] ki[k]`` (:122-140), ``dKI[idx_k] += sum_g ds[g,k] qi[g]``
  scatter-added per slot (:142-162).

All fp32 (the golden's ``astype(float16).astype(float32)`` input rounding is the
io dtype of the inputs here). Returns (d_query_index, d_key_index, d_weights, loss)
rounded to the inputs' dtypes (loss fp32).
"""
import numpy as np

from .sparse_flash_attention_ref import _round_io

EPS = 1e-8


def sli_grad_kl_loss(q, k, qr, kr, qi, ki, w, si, sm_max, sm_sum, scale, act_q=None, act_k=None,
                     io_dtype="fp16", w_dtype=None):
    f = lambda x: np.asarray(x, np.float32)
    q, k, qr, kr, qi, ki, w = (f(x) for x in (q, k, qr, kr, qi, ki, w))
    sm_max, sm_sum = f(sm_max), f(sm_sum)
    si = np.asarray(si, np.int64)
    B, S1, N1, D = q.shape
    S2 = k.shape[1]
    Nidx1, Didx = qi.shape[2], qi.shape[3]
    topK = si.shape[3]
    act_q = np.full(B, S1) if act_q is None else np.asarray(act_q)
    act_k = np.full(B, S2) if act_k is None else np.asarray(act_k)
    dqi = np.zeros_like(qi)
    dki = np.zeros((B, S2, 1, Didx), np.float32)
    dw = np.zeros((B, S1, Nidx1), np.float32)
    loss = 0.0
    for b in range(B):
        aq, ak = int(act_q[b]), int(act_k[b])
        for s1 in range(min(aq, S1)):
            n = min(topK, max(ak - aq + s1 + 1, 0))
            if n <= 0:
                continue
            idx = np.clip(si[b, s1, 0, :n], 0, S2 - 1)
            kg, krg, kig = k[b, idx, 0, :], kr[b, idx, 0, :], ki[b, idx, 0, :]
            scores = (q[b, s1] @ kg.T + qr[b, s1] @ krg.T) * np.float32(scale)           # [N1, n]
            probs = np.exp(scores - sm_max[b, 0, s1][:, None]) / (sm_sum[b, 0, s1][:, None] + EPS)
            p = probs.sum(axis=0) * np.float32(1.0 / N1)                                # [n]
            relu = np.maximum(qi[b, s1] @ kig.T, 0.0)                                  # [Nidx1, n]
            ii = w[b, s1] @ relu                                                       # [n]
            e = np.exp(ii - ii.max())
            si_ = e / (e.sum() + EPS)
            di = si_ - p
            pv, sv = np.maximum(p, EPS), np.maximum(si_, EPS)
            loss += float(np.sum(pv * (np.log(pv) - np.log(sv))))
            dw[b, s1] = relu @ di
            ds = (di[None, :] * w[b, s1][:, None]) * (relu > 0)                         # [Nidx1, n]
            dqi[b, s1] = ds @ kig
            np.add.at(dki[b, :, 0, :], idx, ds.T @ qi[b, s1])
    return (_round_io(dqi, io_dtype), _round_io(dki, io_dtype), _round_io(dw, w_dtype or io_dtype),
            np.array([loss], np.float32))
