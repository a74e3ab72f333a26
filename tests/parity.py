"""Parity helpers: compare the HIP path against the oracle.

Top-k rule (the lightning_indexer parity bar): the golden orders
bf16/fp16-QUANTISED fp32 scores. Two correct fp32 evaluations (numpy BLAS vs
MFMA) of a score x differ by fp32 rounding noise, so they may quantise to
different 16-bit values when x lies close to a rounding boundary. Per element,
with x the float64 score and E an estimate of the fp32 error of a sum of the
score's products (6 sigma of a random-walk model, ``row_error_bound``), the
ADMISSIBLE values are the 16-bit values in [q(x - E), q(x + E)]. A GPU row is
accepted iff
  * every GPU value is admissible for its index (and the oracle's own value is
    admissible too -- a check on E itself), and
  * re-running the golden ordering (oracle.select_topk) with the GPU values on
    the GPU's indices and the LOWEST admissible value everywhere else reproduces
    the GPU's indices AND values exactly.
When E is far below the quantisation step (the usual case) every element has
one admissible value and this is bit-exact equality of the ordered index list.
"""
from __future__ import annotations

import numpy as np

from oracle import lightning_indexer_ref as LI
from oracle.numerics import quantize


def _next16(v32, direction, value_dtype):
    if value_dtype == "fp16":
        h = v32.astype(np.float16)
        return np.nextafter(h, np.float16(np.inf if direction > 0 else -np.inf)).astype(np.float32)
    u = v32.view(np.uint32).astype(np.int64)
    hi = u >> 16
    neg = (hi & 0x8000) != 0
    zero = (hi & 0x7FFF) == 0
    # step magnitude up (away from zero) or down (towards zero) in sign-magnitude bits
    if direction > 0:
        nh = np.where(neg, np.where(zero, 0x0001, hi - 1), hi + 1)
    else:
        nh = np.where(neg, hi + 1, np.where(zero, 0x8001, hi - 1))
    return ((nh.astype(np.uint32) & 0xFFFF) << 16).astype(np.uint32).view(np.float32)


def neighbours(x64, value_dtype):
    """16-bit grid neighbours lo <= x <= hi of float64 values (lo == hi if exact)."""
    x32 = x64.astype(np.float32)
    r = quantize(x32, value_dtype)
    up = _next16(r, +1, value_dtype)
    dn = _next16(r, -1, value_dtype)
    r64 = r.astype(np.float64)
    lo = np.where(r64 <= x64, r, dn)
    hi = np.where(r64 >= x64, r, up)
    return lo, hi


class LiParityStats:
    def __init__(self):
        self.rows = 0
        self.exact_rows = 0
        self.flip_rows = 0
        self.flips = 0
        self.elements = 0          # selected elements checked
        self.gap_rows = 0          # rows whose k-th / (k+1)-th gap exceeds 1e-3 relative
        self.gap_set_mismatch = 0  # of those, rows whose index SET differs (only via flips)

    def __repr__(self):
        return (f"rows={self.rows} exact={self.exact_rows} flip_rows={self.flip_rows} "
                f"flips={self.flips}/{self.elements} "
                f"gap_rows={self.gap_rows} gap_set_mismatch={self.gap_set_mismatch}")


ERR_SIGMAS = 6.0
U32 = 2.0 ** -24


def row_error_bound(q, k, w, b, s1, n2):
    """Per-score fp32 error estimate of one row (float64 [S2]).

    dot_g = sum_d q_gd k_d accumulated in fp32 has error ~ u * sqrt(D/2) * ||q_g o k||_2
    (random walk of the partial sums); the head sum adds ~ u * sqrt(G/2) * ||relu(dot) w||_2.
    Returns ERR_SIGMAS times the root-sum-square of both."""
    N1, N2 = q.shape[2], k.shape[2]
    G = N1 // N2
    D = q.shape[3]
    qg = q[b, s1, n2 * G:(n2 + 1) * G].astype(np.float64)
    kk = k[b, :, n2, :].astype(np.float64)
    wg = w[b, s1, n2 * G:(n2 + 1) * G].astype(np.float64)
    dots = kk @ qg.T                                   # [S2, G]
    act = dots > 0
    qk2 = (kk * kk) @ (qg * qg).T                      # ||q_g o k||^2
    t1 = (D / 2.0) * ((qk2 * act) @ (wg * wg))
    t2 = (G / 2.0) * ((np.maximum(dots, 0) ** 2) @ (wg * wg))
    return ERR_SIGMAS * U32 * np.sqrt(t1 + t2 + (D + G) * 1e-30)


def check_li_row(gpu_idx, gpu_val, s32, s64, act_k, k, value_dtype, stats, err=None,
                 return_value=True, where=""):
    """Check one (b, s1, n2) row. s32 / s64: masked oracle scores (-inf outside);
    err: per-element fp32 error bound (default: 2e-5 relative)."""
    stats.rows += 1
    sq = quantize(s32, value_dtype)
    o_idx, o_val = LI.select_topk(sq, act_k, k)
    # north-star bookkeeping: rows whose k-th / (k+1)-th gap exceeds 1e-3 relative
    order = np.lexsort((np.arange(sq.size), -sq))
    fin = sq[order][np.isfinite(sq[order])]
    if fin.size > k and abs(fin[k - 1]) > 0 and (fin[k - 1] - fin[k]) > 1e-3 * abs(fin[k - 1]):
        stats.gap_rows += 1
        if set(o_idx[o_idx >= 0].tolist()) != set(gpu_idx[gpu_idx >= 0].tolist()):
            stats.gap_set_mismatch += 1
    stats.elements += int((o_idx >= 0).sum())
    gv = gpu_val if return_value else o_val
    if np.array_equal(gpu_idx, o_idx) and (not return_value or np.array_equal(gv, o_val)):
        stats.exact_rows += 1
        return
    assert return_value, f"{where}: index mismatch and no values to explain it"
    assert np.array_equal(gpu_idx >= 0, o_idx >= 0), f"{where}: valid-slot count differs"
    valid = np.isfinite(s64)
    x = np.where(valid, s64, 0.0)
    if err is None:
        err = 2e-5 * np.abs(x)
    amin = quantize((x - err).astype(np.float32), value_dtype)
    amax = quantize((x + err).astype(np.float32), value_dtype)
    # E must cover the golden's own fp32 evaluation
    okq = ~valid | ((sq >= amin) & (sq <= amax))
    assert okq.all(), (f"{where}: error bound too tight for the oracle itself at "
                       f"{np.flatnonzero(~okq)[:5]}")
    out = gpu_idx >= 0
    gi = gpu_idx[out]
    gvv = gv[out]
    assert np.all((gi >= 0) & (gi < sq.size)), f"{where}: index out of range"
    assert np.all(valid[gi]), f"{where}: GPU selected a masked position"
    bad = (gvv < amin[gi]) | (gvv > amax[gi])
    assert not bad.any(), (f"{where}: value outside the fp32 error bound: idx={gi[bad][:5]} "
                           f"gpu={gvv[bad][:5]} oracle={sq[gi][bad][:5]} f64={s64[gi][bad][:5]} "
                           f"E={err[gi][bad][:5]}")
    adj = np.where(valid, amin, sq)
    adj[gi] = gvv
    a_idx, a_val = LI.select_topk(adj, act_k, k)
    assert np.array_equal(a_idx, gpu_idx) and np.array_equal(a_val, gv), (
        f"{where}: GPU order is not the golden order under any admissible rounding: "
        f"first diff at {np.argmax(a_idx != gpu_idx)}")
    stats.flip_rows += 1
    stats.flips += int((gvv != sq[gi]).sum()) + int((~np.isin(o_idx[o_idx >= 0], gi)).sum())


def check_li(gpu_idx, gpu_val, q, k, w, act_q, act_k, sparse_count, sparse_mode, value_dtype,
             rows=None, return_value=True):
    """Compare BSND-shaped GPU outputs [B,S1,N2,k] with the oracle on ``rows``
    (list of (b, s1); default all). q/k/w: fp32 numpy arrays (BSND)."""
    B, S1, N1, D = q.shape
    N2 = k.shape[2]
    if rows is None:
        rows = [(b, s) for b in range(B) for s in range(S1)]
    stats = LiParityStats()
    for b, s1 in rows:
        for n2 in range(N2):
            gi = gpu_idx[b, s1, n2]
            gv = gpu_val[b, s1, n2] if return_value else None
            if s1 >= int(act_q[b]):
                assert np.all(gi == -1), f"row ({b},{s1}) beyond act_q must be all -1"
                if return_value:
                    assert np.all(gv == 0)
                continue
            s32 = LI.li_row_scores(q, k, w, b, s1, n2, act_q, act_k, sparse_mode)
            s64 = LI.li_row_scores_f64(q, k, w, b, s1, n2, act_q, act_k, sparse_mode)
            err = row_error_bound(q, k, w, b, s1, n2)
            check_li_row(gi, gv, s32, s64, int(act_k[b]), sparse_count, value_dtype, stats,
                         err=err, return_value=return_value, where=f"row ({b},{s1},{n2})")
    return stats


def check_topk_properties(idx, val, L_rows, k):
    """Size-independent invariants over ALL rows: the first min(L, k) slots hold
    distinct indices in [0, L), the rest -1 / 0; values non-increasing with ties
    in ascending index order. idx [R, k] int32, val [R, k] fp32, L_rows [R]."""
    R = idx.shape[0]
    nexp = np.minimum(L_rows, k)
    slot = np.arange(k)[None, :]
    validm = slot < nexp[:, None]
    assert np.all((idx >= 0) == validm), "valid-slot prefix length != min(L, k)"
    assert np.all(val[~validm] == 0), "padding slots must hold value 0"
    assert np.all(idx[validm] < np.repeat(L_rows, nexp)), "index outside the visible prefix"
    vi = np.where(validm, val, -np.inf)
    dv = vi[:, 1:] - vi[:, :-1]
    both = validm[:, 1:]
    assert np.all(dv[both] <= 0), "values not non-increasing"
    ties = both & (dv == 0)
    di = idx[:, 1:].astype(np.int64) - idx[:, :-1]
    assert np.all(di[ties] > 0), "ties not in ascending index order"
    s = np.sort(np.where(validm, idx, -1 - slot), axis=1)
    assert np.all(s[:, 1:] != s[:, :-1]), "duplicate indices in a row"
