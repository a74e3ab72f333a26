"""GPU parity of the chained DSA prefill step (dsa_triton_ascend_amd/pipeline.py):
lightning_indexer on packed TND sequences feeding sparse_flash_attention in place
(BASELINE config 5 shape family).

The indexer's indices are checked like tests/test_li_gpu.py::test_tnd (exact, or
the rounding-aware row rule of tests/parity.py); the attention output is checked
against the oracle run on the GPU's own indices, so a legitimate top-k tie flip
cannot fail the attention check.
"""
import numpy as np
import pytest
import torch

from dsa_triton_ascend_amd import PrefillPlan
from dsa_triton_ascend_amd import workloads as W
from oracle import lightning_indexer_ref as LI
from oracle import sparse_flash_attention_ref as SFA
from tests.parity import LiParityStats, check_li_row, check_topk_properties, row_error_bound
from tests.test_sfa_gpu import ROW_REL_TOL, row_rel_err

pytestmark = pytest.mark.gpu

OUT_TOL = dict(rtol=1e-2, atol=1e-2)
LSE_TOL = dict(rtol=1e-4, atol=1e-5)


def _np(t):
    return t.float().cpu().numpy()


def _seq(t, start, L):
    """Sequence b of a packed [T, ...] tensor as a float32 [1, L, ...] array (no padding)."""
    return _np(t[start:start + L])[None]


def _check_indexer_rows(inp, idx, val, lens, k, rows_by_seq):
    gi, gv = idx.cpu().numpy(), val.float().cpu().numpy()
    stats = LiParityStats()
    start = 0
    for L, rows in zip(lens, rows_by_seq):
        qb = _seq(inp["index_query"], start, L)
        kb = _seq(inp["index_key"], start, L)
        wb = _seq(inp["index_weights"], start, L)
        act = np.array([L], np.int32)
        for s in rows:
            s32 = LI.li_row_scores(qb, kb, wb, 0, s, 0, act, act, 3)
            s64 = LI.li_row_scores_f64(qb, kb, wb, 0, s, 0, act, act, 3)
            err = row_error_bound(qb, kb, wb, 0, s, 0)
            check_li_row(gi[start + s, 0], gv[start + s, 0], s32, s64, L, k, "bf16", stats, err=err)
        start += L
    assert stats.flips <= max(4, 0.02 * stats.elements), stats
    return stats


def _check_attention_rows(inp, idx, out, smax, ssum, lens, rows_by_seq):
    """Oracle SFA on the GPU's own indices. Row s of a causal sequence is a one-row
    problem over the key prefix [0, s]: act_q = 1, act_k = s + 1 gives the same
    threshold s + 1 as the full mode-3 row."""
    idx_np = idx.cpu().numpy()
    go, gm, gs = _np(out), _np(smax)[0], _np(ssum)[0]
    start = 0
    for L, rows in zip(lens, rows_by_seq):
        kb = _seq(inp["key"], start, L)
        krb = _seq(inp["key_rope"], start, L)
        for s in rows:
            r = start + s
            q = _np(inp["query"][r:r + 1])[None]
            qr = _np(inp["query_rope"][r:r + 1])[None]
            si = idx_np[r:r + 1][None]
            o_out, o_max, o_sum = SFA.sfa_golden_bsnd(q, kb, si, qr, krb, inp["scale_value"],
                                                      np.array([1], np.int32), np.array([s + 1], np.int32),
                                                      1, 3, "bf16")
            assert np.all(np.isfinite(go[r]))
            np.testing.assert_allclose(go[r], o_out[0, 0], err_msg=f"pipeline row {r}: attention_out", **OUT_TOL)
            rel = row_rel_err(go[r], o_out[0, 0])
            assert rel <= ROW_REL_TOL, f"pipeline row {r}: per-head relative error {rel:.3e} > {ROW_REL_TOL}"
            np.testing.assert_allclose(gm[r], o_max[0, 0, 0], err_msg=f"pipeline row {r}: softmax_max", **LSE_TOL)
            np.testing.assert_allclose(gs[r], o_sum[0, 0, 0], err_msg=f"pipeline row {r}: softmax_sum", **LSE_TOL)
        start += L


def _run(lens, N_idx, N1, k, seed, dev):
    inp = W.tnd_pipeline_inputs(lengths=lens, N_idx=N_idx, N1=N1, sparse_count=k, device="cpu", seed=seed)
    d = {n: (t.to(dev) if torch.is_tensor(t) and n != "cu_seqlens" else t) for n, t in inp.items()}
    cu = inp["cu_seqlens"].tolist()
    plan = PrefillPlan(d["index_query"], d["index_key"], d["index_weights"], d["query"], d["key"],
                       d["query_rope"], d["key_rope"], cu, sparse_count=k, scale_value=inp["scale_value"],
                       return_softmax_lse=True, return_value=True)
    idx, out, smax, ssum = plan.run()
    torch.cuda.synchronize()
    return inp, cu, idx, plan.values, out, smax, ssum


def test_prefill_pipeline_small(dev):
    lens, k = [64, 200, 37, 300], 64
    inp, cu, idx, val, out, smax, ssum = _run(lens, 8, 16, k, 5, dev)
    T = sum(lens)
    assert idx.shape == (T, 1, k) and out.shape == (T, 16, 512) and smax.shape == (1, T, 16)
    rows = [range(L) for L in lens]
    _check_indexer_rows(inp, idx, val, lens, k, rows)
    _check_attention_rows(inp, idx, out, smax, ssum, lens, rows)


@pytest.mark.slow
def test_prefill_pipeline_c5_sampled(dev):
    """BASELINE config 5 at full size: 18216 packed rows, 64 indexer heads, top-2048,
    128 attention heads. Top-k invariants on every row; oracle parity on rows that
    cover every sequence, both ends and the causal ramp."""
    lens, k = list(W.C5_LENGTHS), 2048
    inp, cu, idx, val, out, smax, ssum = _run(lens, 64, 128, k, 42, dev)
    T = sum(lens)
    L_rows = np.concatenate([np.arange(1, L + 1) for L in lens])
    check_topk_properties(idx.cpu().numpy()[:, 0], val.float().cpu().numpy()[:, 0], L_rows, k)
    assert torch.isfinite(out.float()).all()
    rows = [sorted({0, 1, L // 3, min(2047, L - 1), L - 1}) for L in lens]
    _check_indexer_rows(inp, idx, val, lens, k, rows)
    # attention: 24 rows per sequence spread evenly over the causal ramp, plus both ends
    # and the rows around the 2048-token top-k boundary
    att = [sorted({int(x) for x in np.linspace(0, L - 1, 24)} | {0, 1, min(2047, L - 1), min(2048, L - 1), L - 1})
           for L in lens]
    assert all(len(r) >= 16 for r in att)
    _check_attention_rows(inp, idx, out, smax, ssum, lens, att)
