"""GPU parity: the dense lightning-indexer softmax LSE and KL loss backward (HIP) vs
the oracle (oracle/dense_loss_ref.py).

Shape matrix of the reference's tests (test_dense_loss_backward_triton.py:20-60):
B=1, S1 in {2,3,4}, S2 in {64,96,128}, N1 = N2 = 32 (the grouped-head teacher),
D, D_idx in {128,256,512}, Nidx1 in {32,64,128}, fp16 / bf16 inputs from
randn -> fp16 -> dtype (:169-177), weights |randn|, attention stats from full
causal attention (:180-214). Tolerances are the reference's (:62-108): atol / rtol
1e-2 for 16-bit outputs, 1e-3 for float32, with its ratio budget (pass when the
fraction of elements beyond the bound is below rtol). Also N2 = 1 (the MFMA
teacher), grouped heads with G = 4, actual lengths, no rope, omitted index stats,
a row with sum_index <= 0, and the reference's perf shape (B=1, S1=512, S2=4096,
N1 = N2 = 64, D = 128, Nidx1 = 64, D_idx = 128) on a strided sample of rows, and the
full perf-shape call against single-row calls (bit-exact per row).
"""
import math

import numpy as np
import pytest
import torch

from dsa_triton_ascend_amd import dense_lightning_indexer_softmax_lse, dense_loss_backward
from oracle import dense_loss_ref as DLO

pytestmark = pytest.mark.gpu

DT = {"bf16": torch.bfloat16, "fp16": torch.float16}


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available()
    return torch.device("cuda:0")


def _np(t):
    return t.float().cpu().numpy()


def _ratio_close(name, got, want, tol):
    """The reference's comparison (test_dense_loss_backward_triton.py:80-108)."""
    assert np.all(np.isfinite(got)), f"{name}: not finite"
    err = np.abs(got - want)
    bad = np.greater(err, tol + np.abs(got) * tol)
    ratio = bad.sum() / max(bad.size, 1)
    assert ratio < tol, f"{name}: {bad.sum()}/{bad.size} beyond atol=rtol={tol}, max err {err.max():.3e}"


def _inputs(B, S1, S2, N1, N2, D, Nidx1, Didx, dtype, seed=0, rope=True):
    rng = np.random.RandomState(seed)
    t = lambda *s: torch.from_numpy(rng.randn(*s).astype(np.float16)).to(DT[dtype])
    q, k = t(B, S1, N1, D), t(B, S2, N2, D)
    qr, kr = (t(B, S1, N1, 64), t(B, S2, N2, 64)) if rope else (None, None)
    qi, ki = t(B, S1, Nidx1, Didx), t(B, S2, 1, Didx)
    w = torch.from_numpy(np.abs(rng.randn(B, S1, Nidx1)).astype(np.float16)).to(DT[dtype])
    return q, k, qr, kr, qi, ki, w


def _attn_stats(q, k, qr, kr, scale, act_q=None, act_k=None):
    """Full causal attention stats [B, N2, S1, G] (test_dense_loss_backward_triton.py:180-214)."""
    q, k = _np(q), _np(k)
    qr = None if qr is None else _np(qr)
    kr = None if kr is None else _np(kr)
    B, S1, N1, _ = q.shape
    S2, N2 = k.shape[1], k.shape[2]
    G = N1 // N2
    mx = np.full((B, N2, S1, G), -np.inf, np.float32)
    sm = np.zeros((B, N2, S1, G), np.float32)
    for b in range(B):
        aq = S1 if act_q is None else act_q[b]
        ak = S2 if act_k is None else act_k[b]
        for s1 in range(min(S1, aq)):
            lim = min(max(ak - aq + s1 + 1, 0), S2)
            if lim == 0:
                continue
            for h in range(N1):
                sc = q[b, s1, h] @ k[b, :lim, h // G].T
                if qr is not None:
                    sc = sc + qr[b, s1, h] @ kr[b, :lim, h // G].T
                sc = sc * scale
                mx[b, h // G, s1, h % G] = sc.max()
                sm[b, h // G, s1, h % G] = np.exp(sc - sc.max()).sum()
    return mx, sm


def _run(dev, B, S1, S2, N1, N2, D, Nidx1, Didx, dtype, rope=True, act_q=None, act_k=None,
         given_stats=True, seed=0):
    q, k, qr, kr, qi, ki, w = _inputs(B, S1, S2, N1, N2, D, Nidx1, Didx, dtype, seed, rope)
    scale = 1.0 / math.sqrt(D + (64 if rope else 0))
    smx, ssm = _attn_stats(q, k, qr, kr, scale, act_q, act_k)
    g = lambda x: None if x is None else x.to(dev)
    mxi, smi = dense_lightning_indexer_softmax_lse(g(qi), g(ki), g(w), actual_seq_qlen=act_q,
                                                   actual_seq_klen=act_k)
    got = dense_loss_backward(g(q), g(k), g(qi), g(ki), g(w), g(torch.from_numpy(smx)), g(torch.from_numpy(ssm)),
                              mxi if given_stats else None, smi if given_stats else None, scale,
                              query_rope=g(qr), key_rope=g(kr), actual_seq_qlen=act_q, actual_seq_klen=act_k)
    torch.cuda.synchronize()
    want_lse = DLO.dense_softmax_lse(_np(qi), _np(ki), _np(w), act_q, act_k)
    # the golden takes the stats the kernel produced (the reference feeds its own LSE
    # into the backward, test_dense_loss_backward_triton.py:412-425)
    want = DLO.dense_loss_backward(_np(q), _np(k), None if qr is None else _np(qr), None if kr is None else _np(kr),
                                   _np(qi), _np(ki), _np(w), smx, ssm, _np(mxi), _np(smi), scale, act_q, act_k,
                                   io_dtype=dtype)
    return (mxi, smi), want_lse, got, want


def _check(lse, want_lse, got, want, what):
    for name, gv, wv in zip(("softmax_max_index", "softmax_sum_index"), lse, want_lse):
        gv = _np(gv)
        fin = np.isfinite(wv)
        assert np.array_equal(fin, np.isfinite(gv)), f"{what}: {name} -inf rows differ"
        np.testing.assert_allclose(gv[fin], wv[fin], rtol=1e-4, atol=1e-4, err_msg=f"{what}: {name}")
    for name, gv, wv in zip(("d_query_index", "d_key_index", "d_weights"), got[:3], want[:3]):
        _ratio_close(f"{what}: {name}", _np(gv), wv, 1e-2)
    np.testing.assert_allclose(_np(got[3]), want[3], rtol=1e-3, atol=1e-3, err_msg=f"{what}: loss")


CORE = [(1, 2, 64, 32, 32, d, nidx1, didx) for d in (128, 256, 512) for nidx1 in (32, 64, 128)
        for didx in (128, 256, 512)]
# the reference's full core matrix (test_dense_loss_backward_triton.py:20-25, which includes its fp16
# smoke's Nidx1 = 128 x D_idx = 512, :55-60) and its extra shapes (:27-31)
EXTRA = [(1, 3, 96, 32, 32, 128, 32, 128), (1, 4, 128, 32, 32, 128, 32, 128)]


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("B,S1,S2,N1,N2,D,Nidx1,Didx", CORE + EXTRA)
def test_dense_matrix(dev, B, S1, S2, N1, N2, D, Nidx1, Didx, dtype):
    lse, want_lse, got, want = _run(dev, B, S1, S2, N1, N2, D, Nidx1, Didx, dtype)
    _check(lse, want_lse, got, want, f"S1={S1} S2={S2} D={D} Nidx1={Nidx1} D_idx={Didx} {dtype}")


@pytest.mark.parametrize("case", ["long_rows", "long_rows_wide_qi"])
def test_dense_rows_longer_than_4096_keys(dev, case):
    """S2 = 6000: every row sees 5997..6000 keys, past the 4096 index scores the student
    keeps in LDS, so they live in the workspace (the LSE runs its statistics online);
    also with the widest qi block (Nidx1 = 128 x D_idx = 512, taken in two passes)."""
    kw = dict(B=1, S1=4, S2=6000, N1=16, N2=16, D=128, Nidx1=64, Didx=128, dtype="bf16")
    if case == "long_rows_wide_qi":
        kw.update(Nidx1=128, Didx=512, N2=1, dtype="fp16")
    lse, want_lse, got, want = _run(dev, **kw)
    _check(lse, want_lse, got, want, case)


@pytest.mark.parametrize("case", ["mqa", "gqa4", "lengths", "no_rope", "own_stats"])
def test_dense_variants(dev, case):
    kw = dict(B=2, S1=5, S2=200, N1=16, N2=16, D=128, Nidx1=64, Didx=128, dtype="bf16")
    if case == "mqa":
        kw.update(N2=1)
    elif case == "gqa4":
        kw.update(N2=4, D=256)
    elif case == "lengths":
        kw.update(act_q=[5, 3], act_k=[2, 150])   # batch 0: rows 0..2 see no key
    elif case == "no_rope":
        kw.update(rope=False, D=512)
    elif case == "own_stats":
        kw.update(given_stats=False)
    lse, want_lse, got, want = _run(dev, **kw)
    _check(lse, want_lse, got, want, case)


def test_dense_row_with_empty_index_softmax(dev):
    """sum_index <= 0 marks a row without gradient or loss (dense_loss_backward_triton.py:
    246-252): the kernel skips it while its neighbours are unchanged."""
    B, S1, S2, N1, D, Nidx1, Didx = 1, 4, 64, 32, 128, 32, 128
    q, k, qr, kr, qi, ki, w = _inputs(B, S1, S2, N1, N1, D, Nidx1, Didx, "fp16", seed=5)
    scale = 1.0 / math.sqrt(D + 64)
    smx, ssm = _attn_stats(q, k, qr, kr, scale)
    g = lambda x: x.to(dev)
    mxi, smi = dense_lightning_indexer_softmax_lse(g(qi), g(ki), g(w))
    smi[0, 0, 2] = 0.0
    got = dense_loss_backward(g(q), g(k), g(qi), g(ki), g(w), g(torch.from_numpy(smx)), g(torch.from_numpy(ssm)),
                              mxi, smi, scale, query_rope=g(qr), key_rope=g(kr))
    torch.cuda.synchronize()
    want = DLO.dense_loss_backward(_np(q), _np(k), _np(qr), _np(kr), _np(qi), _np(ki), _np(w), smx, ssm,
                                   _np(mxi), _np(smi), scale, io_dtype="fp16")
    assert float(got[0][0, 2].abs().max()) == 0.0 and float(got[2][0, 2].abs().max()) == 0.0
    for name, gv, wv in zip(("dqi", "dki", "dw"), got[:3], want[:3]):
        _ratio_close(name, _np(gv), wv, 1e-2)
    np.testing.assert_allclose(_np(got[3]), want[3], rtol=1e-3)


def test_dense_perf_shape_sampled_rows(dev):
    """The reference's perf shape (perf_dense_loss_backward_triton.py:18), 4096 keys at
    the last row: every 64th query row of S1 = 512 is run as its own S1 = 1 call over
    its causal key range (keys 0 .. 4096 - 512 + s1), kernel and oracle alike."""
    B, S1, S2, N1, N2, D, Nidx1, Didx = 1, 512, 4096, 64, 64, 128, 64, 128
    rows = list(range(63, 512, 64))
    q, k, qr, kr, qi, ki, w = _inputs(B, S1, S2, N1, N2, D, Nidx1, Didx, "bf16", seed=2)
    scale = 1.0 / math.sqrt(D + 64)
    g = lambda x: x.to(dev)
    for s1 in rows:
        lim = S2 - S1 + s1 + 1
        sl = slice(s1, s1 + 1)
        qj, qrj, qij, wj = q[:, sl], qr[:, sl], qi[:, sl], w[:, sl]
        kj, krj, kij = k[:, :lim], kr[:, :lim], ki[:, :lim]
        smx, ssm = _attn_stats(qj, kj, qrj, krj, scale)
        mxi, smi = dense_lightning_indexer_softmax_lse(g(qij), g(kij), g(wj))
        out = dense_loss_backward(g(qj), g(kj), g(qij), g(kij), g(wj), g(torch.from_numpy(smx)),
                                  g(torch.from_numpy(ssm)), mxi, smi, scale, query_rope=g(qrj), key_rope=g(krj))
        torch.cuda.synchronize()
        want = DLO.dense_loss_backward(_np(qj), _np(kj), _np(qrj), _np(krj), _np(qij), _np(kij), _np(wj), smx,
                                       ssm, _np(mxi), _np(smi), scale, io_dtype="bf16")
        for name, gv, wv in zip(("dqi", "dki", "dw"), out[:3], want[:3]):
            _ratio_close(f"row {s1}: {name}", _np(gv), wv, 1e-2)
        np.testing.assert_allclose(_np(out[3]), want[3], rtol=1e-3, err_msg=f"row {s1}: loss")


def test_dense_perf_shape_full_call_matches_single_rows(dev):
    """The full perf-shape call (S1 = 512 at once: 16 row blocks, causal early exits) gives
    every sampled row the d_query_index and d_weights of that row run alone (which the
    test above checks against the oracle), bit for bit: a row's teacher and student do the
    same arithmetic in either arrangement. All four outputs of the full call (d_key_index
    summed over every row, the loss over every row) against the oracle on all 512 rows."""
    B, S1, S2, N1, N2, D, Nidx1, Didx = 1, 512, 4096, 64, 64, 128, 64, 128
    q, k, qr, kr, qi, ki, w = (x.to(dev) for x in _inputs(B, S1, S2, N1, N2, D, Nidx1, Didx, "bf16", seed=4))
    scale = 1.0 / math.sqrt(D + 64)
    gen = torch.Generator(device=dev).manual_seed(1)
    smx = torch.rand(B, N2, S1, 1, device=dev, generator=gen) * 4.0
    ssm = 1.0 + torch.rand(B, N2, S1, 1, device=dev, generator=gen) * 50.0
    mxi, smi = dense_lightning_indexer_softmax_lse(qi, ki, w)
    full = dense_loss_backward(q, k, qi, ki, w, smx, ssm, mxi, smi, scale, query_rope=qr, key_rope=kr)
    torch.cuda.synchronize()
    for s1 in (0, 31, 32, 200, 511):
        lim = S2 - S1 + s1 + 1
        sl = slice(s1, s1 + 1)
        one = dense_loss_backward(q[:, sl], k[:, :lim], qi[:, sl], ki[:, :lim], w[:, sl],
                                  smx[:, :, sl].contiguous(), ssm[:, :, sl].contiguous(), mxi[:, :, sl],
                                  smi[:, :, sl], scale, query_rope=qr[:, sl], key_rope=kr[:, :lim])
        torch.cuda.synchronize()
        assert torch.equal(full[0][:, sl], one[0]), f"row {s1}: d_query_index differs"
        assert torch.equal(full[2][:, sl], one[2]), f"row {s1}: d_weights differs"
    assert torch.isfinite(full[1]).all() and torch.isfinite(full[3]).all()
    # d_key_index sums every row's contribution (fp32 atomics) and the loss is the row-ordered
    # sum of the row losses: both against the oracle over all 512 rows (the LSE stats are the
    # GPU's, which the LSE tests check on their own)
    want = DLO.dense_loss_backward(_np(q), _np(k), _np(qr), _np(kr), _np(qi), _np(ki), _np(w), _np(smx), _np(ssm),
                                   _np(mxi), _np(smi), scale, io_dtype="bf16")
    _ratio_close("full call: dki", _np(full[1]), want[1], 1e-2)
    _ratio_close("full call: dqi", _np(full[0]), want[0], 1e-2)
    _ratio_close("full call: dw", _np(full[2]), want[2], 1e-2)
    np.testing.assert_allclose(_np(full[3]), want[3], rtol=1e-3, err_msg="full call: loss")
    rel = np.linalg.norm(_np(full[1]) - want[1]) / np.linalg.norm(want[1])
    print(f"[dense parity] perf shape d_key_index relative Frobenius error {rel:.2e}")
    assert rel <= 1e-2

