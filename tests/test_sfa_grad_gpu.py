"""GPU parity: sparse_flash_attention_grad (HIP) vs the oracle
(oracle/sparse_flash_attention_grad_ref.py).

Shape matrix follows the reference's test_golden (test_sfa_grad_triton.py:124-189):
token-wise and block-wise (bs 2, 4), S1 = 1, N1 = 1 and 128, topK = 2048, multi-batch,
D in {128, 256, 512}, fp16 / bf16; the forward outputs and stats come from this
library's forward (the reference's fwd_source="triton" leg). Tolerances are the
reference's (test_sfa_grad_triton.py:87-89): rtol 6e-2 / atol 5e-2 (bf16), rtol 3e-2 /
atol 2e-2 (fp16), atol scaled by sqrt(S1) for d_key / d_value / d_key_rope. Also mode 0,
actual lengths, TND, and the linearity of the backward in d_out at the perf shape.
"""
import math

import numpy as np
import pytest
import torch

from dsa_triton_ascend_amd import sparse_flash_attention, sparse_flash_attention_grad
from oracle import sparse_flash_attention_grad_ref as SFG

pytestmark = pytest.mark.gpu

DT = {"bf16": torch.bfloat16, "fp16": torch.float16}


def _np(t):
    return t.float().cpu().numpy()


def _tol(dtype, scale=1.0):
    rtol = 6e-2 if dtype == "bf16" else 3e-2
    atol = (5e-2 if dtype == "bf16" else 2e-2) * scale
    return dict(rtol=rtol, atol=atol)


def _ref_indices(B, S1, S2, count, bs, mode, act_q=None, act_k=None, seed=7):
    """Reference index generator (test_sfa_grad_triton.py:51-68): per row, the first
    min(count, ceil(threshold/bs)) slots hold sorted distinct block ids, the rest -1."""
    rng = np.random.RandomState(seed)
    si = np.full((B, S1, 1, count), -1, dtype=np.int32)
    for b in range(B):
        aq = S1 if act_q is None else act_q[b]
        ak = S2 if act_k is None else act_k[b]
        for s1 in range(S1):
            thr = ak if mode == 0 else ak - aq + s1 + 1
            if thr <= 0:
                continue
            nb = int(np.ceil(thr / bs))
            n = min(count, nb)
            si[b, s1, 0, :n] = np.sort(rng.permutation(nb)[:n]).astype(np.int32)
    return si


def _inputs(B, S1, S2, N1, D, dtype, seed=42):
    """Reference generator semantics (test_sfa_grad_triton.py:71-84): randn -> fp16 -> dtype."""
    rng = np.random.RandomState(seed)
    t = lambda *s: torch.from_numpy(rng.randn(*s).astype(np.float16)).to(DT[dtype])
    q, k, v, qr, kr, do = (t(B, S1, N1, D), t(B, S2, 1, D), t(B, S2, 1, D), t(B, S1, N1, 64),
                           t(B, S2, 1, 64), t(B, S1, N1, D))
    return q, k, v, qr, kr, do


def _check(got, want, dtype, S1, what):
    names = ("d_query", "d_key", "d_value", "d_query_rope", "d_key_rope")
    for name, g, w in zip(names, got, want):
        gv = _np(g)
        assert gv.shape == w.shape, f"{what}: {name} shape {gv.shape} vs {w.shape}"
        assert np.all(np.isfinite(gv)), f"{what}: {name} not finite"
        sc = math.sqrt(S1) if name in ("d_key", "d_value", "d_key_rope") else 1.0
        np.testing.assert_allclose(gv, w, err_msg=f"{what}: {name}", **_tol(dtype, sc))


def _run_case(dev, B, S1, S2, N1, count, bs, mode, D, dtype, act_q=None, act_k=None):
    q, k, v, qr, kr, do = _inputs(B, S1, S2, N1, D, dtype)
    si = _ref_indices(B, S1, S2, count, bs, mode, act_q, act_k)
    scale = 1.0 / math.sqrt(D + 64)
    g = lambda x: x.to(dev)
    out, smax, ssum = sparse_flash_attention(g(q), g(k), g(v), g(torch.from_numpy(si)), scale_value=scale,
                                             actual_seq_lengths_query=act_q, actual_seq_lengths_kv=act_k,
                                             query_rope=g(qr), key_rope=g(kr), sparse_block_size=bs,
                                             sparse_mode=mode, return_softmax_lse=True)
    got = sparse_flash_attention_grad(g(q), g(k), g(v), g(torch.from_numpy(si)), g(do), out, smax, ssum,
                                      scale_value=scale, query_rope=g(qr), key_rope=g(kr),
                                      actual_seq_lengths_query=act_q, actual_seq_lengths_kv=act_k,
                                      sparse_block_size=bs, sparse_mode=mode)
    torch.cuda.synchronize()
    want = SFG.sparse_flash_attention_grad(_np(q), _np(k), None, si, _np(do), _np(out), _np(smax), _np(ssum),
                                           scale, _np(qr), _np(kr), act_q, act_k, bs, "BSND", mode,
                                           io_dtype=dtype)
    return got, want


GOLDEN = [
    (1, 4, 128, 8, 64, 1, 3),       # token-wise, rightDownCausal
    (2, 16, 256, 16, 128, 1, 3),    # bigger, multi-batch
    (1, 8, 128, 8, 32, 2, 3),       # block-wise (block_size=2)
    (1, 8, 256, 16, 32, 4, 3),      # block-wise (block_size=4)
    (1, 1, 128, 8, 16, 1, 3),       # S1=1 single query row
    (1, 4, 128, 1, 64, 1, 3),       # N1=1 single head
    (1, 4, 128, 128, 64, 1, 3),     # N1=128 (four head blocks)
    (1, 4, 2048, 8, 2048, 1, 3),    # topK=2048
    (1, 4, 128, 8, 64, 1, 0),       # full mode (commented out in the reference matrix)
]


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available()
    return torch.device("cuda:0")


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("D", [128, 256, 512])
@pytest.mark.parametrize("B,S1,S2,N1,count,bs,mode", GOLDEN)
def test_grad_golden_matrix(dev, B, S1, S2, N1, count, bs, mode, D, dtype):
    got, want = _run_case(dev, B, S1, S2, N1, count, bs, mode, D, dtype)
    _check(got, want, dtype, S1, f"B{B} S1={S1} S2={S2} N1={N1} k={count} bs={bs} mode={mode} D={D} {dtype}")


def test_grad_actual_lengths_and_skips(dev):
    """act_q < S1 (rows past it untouched: zero gradients), act_k < S2 (keys past it get
    nothing), mode-3 leading rows with s1 < act_q - act_k skipped."""
    B, S1, S2, N1, D, count = 2, 12, 64, 16, 256, 48
    act_q, act_k = [12, 9], [5, 40]
    got, want = _run_case(dev, B, S1, S2, N1, count, 1, 3, D, "bf16", act_q, act_k)
    _check(got, want, "bf16", S1, "actual lengths")
    assert float(got[0][1, 9:].abs().max()) == 0.0        # rows past act_q
    assert float(got[1][0, 5:].abs().max()) == 0.0        # keys past act_k of batch 0


def test_grad_tnd(dev):
    """TND: packed rows of three batches, cumulative lengths, stats (1, T1, N1)."""
    lq, lk = [3, 5, 2], [40, 96, 64]
    T1, T2, N1, D, count, dtype = sum(lq), sum(lk), 32, 512, 64, "bf16"
    rng = np.random.RandomState(9)
    t = lambda *s: torch.from_numpy(rng.randn(*s).astype(np.float16)).to(DT[dtype])
    q, qr, do = t(T1, N1, D), t(T1, N1, 64), t(T1, N1, D)
    k, kr = t(T2, 1, D), t(T2, 1, 64)
    si = np.full((T1, 1, count), -1, np.int32)
    row = 0
    for b in range(3):
        for s1 in range(lq[b]):
            thr = lk[b] - lq[b] + s1 + 1
            n = min(count, thr)
            si[row, 0, :n] = np.sort(rng.permutation(thr)[:n])
            row += 1
    cq, ck = np.cumsum(lq).tolist(), np.cumsum(lk).tolist()
    scale = 1.0 / math.sqrt(D + 64)
    g = lambda x: x.to(dev)
    out, smax, ssum = sparse_flash_attention(g(q), g(k), g(k), g(torch.from_numpy(si)), scale_value=scale,
                                             actual_seq_lengths_query=cq, actual_seq_lengths_kv=ck,
                                             query_rope=g(qr), key_rope=g(kr), layout_query="TND",
                                             layout_kv="TND", sparse_mode=3, return_softmax_lse=True)
    got = sparse_flash_attention_grad(g(q), g(k), g(k), g(torch.from_numpy(si)), g(do), out, smax, ssum,
                                      scale_value=scale, query_rope=g(qr), key_rope=g(kr),
                                      actual_seq_lengths_query=cq, actual_seq_lengths_kv=ck,
                                      layout="TND", sparse_mode=3)
    torch.cuda.synchronize()
    want = SFG.sparse_flash_attention_grad(_np(q), _np(k), None, si, _np(do), _np(out), _np(smax), _np(ssum),
                                           scale, _np(qr), _np(kr), cq, ck, 1, "TND", 3, io_dtype=dtype)
    _check(got, want, dtype, max(lq), "TND")


def test_grad_perf_shape_all_rows(dev):
    """The reference's grad perf shape (perf_sfa_grad_triton.py:23: B=1, S1=512, S2=4096, N1=64,
    topK=2048, D=512, bf16) against the oracle on all 512 rows: every key row's d_key / d_value
    sums the contributions of every query row that selects it. Elementwise: the reference's bf16
    tolerances (atol scaled by sqrt(S1) for the key-side sums); on top of that each gradient
    within 2e-2 of the oracle in relative Frobenius norm."""
    B, S1, S2, N1, D, count = 1, 512, 4096, 64, 512, 2048
    q, k, v, qr, kr, do = _inputs(B, S1, S2, N1, D, "bf16", seed=3)
    si = _ref_indices(B, S1, S2, count, 1, 3)
    scale = 1.0 / math.sqrt(D + 64)
    g = lambda x: x.to(dev)
    out, smax, ssum = sparse_flash_attention(g(q), g(k), g(k), g(torch.from_numpy(si)), scale_value=scale,
                                             query_rope=g(qr), key_rope=g(kr), sparse_mode=3,
                                             return_softmax_lse=True)
    got = sparse_flash_attention_grad(g(q), g(k), g(k), g(torch.from_numpy(si)), g(do), out, smax, ssum,
                                      scale_value=scale, query_rope=g(qr), key_rope=g(kr), sparse_mode=3)
    torch.cuda.synchronize()
    want = SFG.sparse_flash_attention_grad(_np(q), _np(k), None, si, _np(do), _np(out), _np(smax), _np(ssum),
                                           scale, _np(qr), _np(kr), None, None, 1, "BSND", 3, io_dtype="bf16")
    _check(got, want, "bf16", S1, "grad perf shape, all rows")
    for name, gv, w in zip(("d_query", "d_key", "d_value", "d_query_rope", "d_key_rope"), got, want):
        rel = np.linalg.norm(_np(gv) - w) / np.linalg.norm(w)
        print(f"[grad parity] perf shape {name}: relative Frobenius error {rel:.2e}")
        assert rel <= 2e-2, f"{name}: relative error {rel:.3e}"


def test_grad_linear_in_d_out_at_perf_shape(dev):
    """Perf shape of the reference (perf_sfa_grad_triton.py:23: B=1, S1=512, S2=4096, N1=64,
    topK=2048, D=512, bf16): the backward is linear in d_out for a fixed forward, so
    grad(a) + grad(b) == grad(a + b) up to rounding; every key row gets contributions
    from hundreds of query rows (the atomics under contention)."""
    B, S1, S2, N1, D, count = 1, 512, 4096, 64, 512, 2048
    q, k, v, qr, kr, do = _inputs(B, S1, S2, N1, D, "bf16", seed=3)
    si = _ref_indices(B, S1, S2, count, 1, 3)
    g = lambda x: x.to(dev)
    q, k, qr, kr, do, sit = g(q), g(k), g(qr), g(kr), g(do), g(torch.from_numpy(si))
    scale = 1.0 / math.sqrt(D + 64)
    out, smax, ssum = sparse_flash_attention(q, k, k, sit, scale_value=scale, query_rope=qr, key_rope=kr,
                                             sparse_mode=3, return_softmax_lse=True)
    do2 = torch.flip(do, dims=[2])
    run = lambda d: sparse_flash_attention_grad(q, k, k, sit, d, out, smax, ssum, scale_value=scale,
                                                query_rope=qr, key_rope=kr, sparse_mode=3)
    ga, gb = [x.float() for x in run(do)], [x.float() for x in run(do2)]
    gab = [x.float() for x in run((do.float() + do2.float()).to(torch.bfloat16))]
    for name, a, b, ab in zip(("dq", "dk", "dv", "dqr", "dkr"), ga, gb, gab):
        assert torch.isfinite(ab).all(), name
        ref = a + b
        err = (ab - ref).abs().max().item()
        assert err <= 2e-2 * ref.abs().max().item() + 1e-3, f"{name}: linearity error {err}"


@pytest.mark.parametrize("N1,D", [(16, 256), (8, 128), (4, 512)])
def test_grad_poisoned_workspace(dev, N1, D):
    """Every element of the dense dS^T / P^T buffers that the library products read is
    written by the call itself (values at the selected tokens, zeros elsewhere, by the
    rows kernel when N1 % 8 == 0, else by clear kernels): a workspace filled with NaN
    bytes beforehand gives the same gradients bit for bit as a fresh one."""
    from dsa_triton_ascend_amd.sparse_flash_attention_grad import GradPlan, INT64_MAX
    B, S1, S2, count = 2, 8, 256, 64
    q, k, v, qr, kr, do = _inputs(B, S1, S2, N1, D, "bf16", seed=11)
    si = _ref_indices(B, S1, S2, count, 1, 3, seed=5)
    scale = 1.0 / math.sqrt(D + 64)
    g = lambda x: x.to(dev)
    q, k, qr, kr, do, sit = g(q), g(k), g(qr), g(kr), g(do), g(torch.from_numpy(si))
    out, smax, ssum = sparse_flash_attention(q, k, k, sit, scale_value=scale, query_rope=qr, key_rope=kr,
                                             sparse_mode=3, return_softmax_lse=True)
    plan = lambda: GradPlan(q, k, k, sit, do, out, smax, ssum, scale, qr, kr, None, None, 1, "BSND", 3,
                            INT64_MAX, INT64_MAX, False)
    clean = plan()
    clean.ws.zero_()
    want = [x.clone() for x in clean.run()]
    dirty = plan()
    dirty.ws.fill_(0xFF)
    got = dirty.run()
    torch.cuda.synchronize()
    for name, a, b in zip(("dq", "dk", "dv", "dqr", "dkr"), got, want):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"N1={N1} D={D}: {name} differs"


def test_grad_nan_in_inactive_rows_does_not_leak(dev):
    """Rows past act_q take no part in the backward (the reference masks them, row_active at
    sparse_flash_attention_grad_triton.py:229): NaN in their q, q_rope and d_out must leave
    every gradient of the batch finite and bit-identical to a run with finite values there."""
    B, S1, S2, N1, D, count = 2, 12, 256, 16, 512, 64
    act_q, act_k = [9, 12], [200, 256]
    q, k, v, qr, kr, do = _inputs(B, S1, S2, N1, D, "bf16", seed=17)
    si = _ref_indices(B, S1, S2, count, 1, 3, act_q, act_k, seed=4)
    scale = 1.0 / math.sqrt(D + 64)
    g = lambda x: x.to(dev)
    k, kr, sit = g(k), g(kr), g(torch.from_numpy(si))

    def run(qq, qqr, ddo):
        out, smax, ssum = sparse_flash_attention(qq, k, k, sit, scale_value=scale, actual_seq_lengths_query=act_q,
                                                 actual_seq_lengths_kv=act_k, query_rope=qqr, key_rope=kr,
                                                 sparse_mode=3, return_softmax_lse=True)
        grads = sparse_flash_attention_grad(qq, k, k, sit, ddo, out, smax, ssum, scale_value=scale, query_rope=qqr,
                                            key_rope=kr, actual_seq_lengths_query=act_q,
                                            actual_seq_lengths_kv=act_k, sparse_mode=3)
        torch.cuda.synchronize()
        return [x.clone() for x in grads]

    clean = run(g(q), g(qr), g(do))
    qn, qrn, don = g(q), g(qr), g(do)
    qn[0, 9:] = float("nan")     # rows past act_q of batch 0
    qrn[0, 9:] = float("nan")
    don[0, 9:] = float("nan")
    dirty = run(qn, qrn, don)
    for name, a, b in zip(("dq", "dk", "dv", "dqr", "dkr"), dirty, clean):
        assert torch.isfinite(a.float()).all(), f"{name}: NaN leaked"
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"{name} differs"


_REPRO_SCRIPT = r"""
import sys, math, numpy as np, torch
sys.path.insert(0, sys.argv[1])
from tests.test_sfa_grad_gpu import _inputs, _ref_indices
from dsa_triton_ascend_amd import sparse_flash_attention, sparse_flash_attention_grad
dev = torch.device("cuda:0")
B, S1, S2, N1, D, count = 1, 512, 4096, 64, 512, 2048
q, k, v, qr, kr, do = _inputs(B, S1, S2, N1, D, "bf16", seed=3)
si = _ref_indices(B, S1, S2, count, 1, 3)
scale = 1.0 / math.sqrt(D + 64)
g = lambda x: x.to(dev)
out, smax, ssum = sparse_flash_attention(g(q), g(k), g(k), g(torch.from_numpy(si)), scale_value=scale,
                                         query_rope=g(qr), key_rope=g(kr), sparse_mode=3, return_softmax_lse=True)
dq, dk, dv, dqr, dkr = sparse_flash_attention_grad(g(q), g(k), g(k), g(torch.from_numpy(si)), g(do), out, smax,
                                                   ssum, scale_value=scale, query_rope=g(qr), key_rope=g(kr),
                                                   sparse_mode=3)
torch.cuda.synchronize()
np.savez(sys.argv[2], **{n: t.view(torch.int16).cpu().numpy() for n, t in
                        zip(("dq", "dk", "dv", "dqr", "dkr"), (dq, dk, dv, dqr, dkr))})
print("saved", flush=True)
"""


def test_grad_bitwise_reproducible_across_processes(tmp_path):
    """The library GEMMs' algorithm is fixed per shape (no per-process timing), so two fresh
    processes produce the same gradient bits at the reference's grad perf shape
    (perf_sfa_grad_triton.py:23)."""
    import subprocess
    import sys
    from pathlib import Path
    root = str(Path(__file__).resolve().parents[1])
    files = []
    for i in range(2):   # one after the other: never more than one extra process on the GPU
        f = tmp_path / f"g{i}.npz"
        r = subprocess.run([sys.executable, "-c", _REPRO_SCRIPT, root, str(f)], capture_output=True, text=True,
                           timeout=240)
        assert r.returncode == 0, r.stderr[-2000:]
        files.append(np.load(f))
    for name in ("dq", "dk", "dv", "dqr", "dkr"):
        assert np.array_equal(files[0][name], files[1][name]), f"{name} differs between processes"
