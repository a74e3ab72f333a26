"""Pins the CPU oracle (oracle/) with checks that do not retype its formulas:
brute force, float64 closed forms, library routines and hand-derived cases.
CPU only (no GPU needed)."""
import math

import numpy as np
import pytest
import torch

from oracle import lightning_indexer_ref as LI
from oracle import sparse_flash_attention_ref as SFA
from oracle.numerics import bf16_bits, bf16_from_bits, quantize, round_bf16, round_fp16
from tests.parity import neighbours, check_li_row, LiParityStats


# ----------------------------------------------------------------- rounding
def test_round_bf16_matches_torch_rne():
    rng = np.random.RandomState(0)
    bits = rng.randint(0, 2**32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    special = np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, 3.4e38, -3.4e38, 1e-40, -1e-40,
                        1.00390625, 1.01171875, 1.005859375, 1.0048828125], dtype=np.float32)
    # exact halfway cases: low 16 bits == 0x8000, both parities of the kept lsb
    half = (np.arange(0x3F80, 0x3F90, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    for arr in (x, special, half):
        want = torch.from_numpy(arr.copy()).to(torch.bfloat16).to(torch.float32).numpy()
        got = round_bf16(arr)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_round_fp16_matches_torch():
    x = np.random.RandomState(1).randn(1 << 16).astype(np.float32) * 100
    want = torch.from_numpy(x).to(torch.float16).to(torch.float32).numpy()
    assert np.array_equal(round_fp16(x), want)
    assert np.isneginf(quantize(np.array([-np.inf], np.float32), "fp16"))[0]
    assert np.isneginf(quantize(np.array([-np.inf], np.float32), "bf16"))[0]


def test_bf16_bits_roundtrip():
    x = round_bf16(np.random.RandomState(2).randn(1000).astype(np.float32))
    assert np.array_equal(bf16_from_bits(bf16_bits(x)), x)


def test_neighbours_bracket():
    x = np.random.RandomState(3).randn(10000) * 10
    for vd in ("bf16", "fp16"):
        lo, hi = neighbours(x, vd)
        assert np.all(lo <= x) and np.all(hi >= x)
        q = quantize(x.astype(np.float32), vd)
        assert np.all((q == lo) | (q == hi))


# ----------------------------------------------------------------- indexer
def _li_inputs(B, S1, S2, N1, N2, D, seed=0):
    rng = np.random.RandomState(seed)
    q = round_bf16(rng.randn(B, S1, N1, D).astype(np.float32))
    k = round_bf16(rng.randn(B, S2, N2, D).astype(np.float32))
    w = rng.randn(B, S1, N1).astype(np.float32)
    return q, k, w


@pytest.mark.parametrize("B,S1,S2,N1,N2,D", [(1, 4, 16, 8, 1, 32), (2, 3, 9, 16, 2, 24),
                                              (1, 5, 7, 7, 1, 12), (1, 6, 3, 12, 4, 8)])
def test_li_scores_closed_form(B, S1, S2, N1, N2, D):
    q, k, w = _li_inputs(B, S1, S2, N1, N2, D)
    G = N1 // N2
    act_q = np.full(B, S1)
    act_k = np.full(B, S2)
    qd, kd, wd = (x.astype(np.float64) for x in (q, k, w))
    for b in range(B):
        for s1 in range(S1):
            for n2 in range(N2):
                got = LI.li_row_scores(q, k, w, b, s1, n2, act_q, act_k, sparse_mode=0)
                dots = np.einsum("gd,sd->gs", qd[b, s1, n2 * G:(n2 + 1) * G], kd[b, :, n2, :])
                want = (np.maximum(dots, 0) * wd[b, s1, n2 * G:(n2 + 1) * G, None]).sum(0)
                np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


def _brute_topk(sq, L, k):
    cand = sorted(((-float(sq[i]), i) for i in range(L) if sq[i] != -np.inf))
    idx = np.full(k, -1, np.int32)
    for j, (_, i) in enumerate(cand[:k]):
        idx[j] = i
    return idx


@pytest.mark.parametrize("mode", [0, 3])
@pytest.mark.parametrize("act", [(6, 20), (8, 6), (1, 20), (6, 6), (0, 5), (8, 0)])
def test_li_golden_brute_force_and_masks(mode, act):
    aq, ak = act
    B, S1, S2, N1, N2, D, K = 1, 8, 20, 4, 2, 16, 7
    q, k, w = _li_inputs(B, S1, S2, N1, N2, D, seed=5)
    # coarse scores create many exact ties after quantisation
    q = round_bf16(np.round(q * 2) / 2)
    k = round_bf16(np.round(k))
    idx, val = LI.li_golden_bsnd(q, k, w, [aq], [ak], K, mode, return_value=True)
    for s1 in range(S1):
        for n2 in range(N2):
            if s1 >= aq:
                assert np.all(idx[0, s1, n2] == -1) and np.all(val[0, s1, n2] == 0)
                continue
            L = min(max(ak - aq + s1 + 1, 0), S2, ak) if mode == 3 else min(ak, S2)
            sq = quantize(LI.li_row_scores(q, k, w, 0, s1, n2, [aq], [ak], mode), "bf16")
            assert np.all(np.isneginf(sq[L:])) and np.all(np.isfinite(sq[:L]))
            want = _brute_topk(sq, L, K)
            assert np.array_equal(idx[0, s1, n2], want), (s1, n2)
            nv = min(L, K)
            assert np.array_equal(val[0, s1, n2, :nv], sq[want[:nv]])
            assert np.all(val[0, s1, n2, nv:] == 0)


def test_li_special_cases():
    q, k, w = _li_inputs(1, 4, 3, 4, 1, 8, seed=9)
    # S1 > S2 with mode 3: row s1 sees min(S2 - S1 + s1 + 1, S2) keys, the first row none
    idx, _ = LI.li_golden_bsnd(q, k, w, [4], [3], 4, 3, return_value=True)
    assert [int((idx[0, s, 0] >= 0).sum()) for s in range(4)] == [0, 1, 2, 3]
    # S1 == 1 with act_q == act_k == 1 sees key 0 only
    idx, _ = LI.li_golden_bsnd(q[:, :1], k, w[:, :1], [1], [1], 2, 3, return_value=True)
    assert idx[0, 0, 0].tolist() == [0, -1]
    # return_value=False gives zeros
    _, val = LI.li_golden_bsnd(q, k, w, [4], [3], 4, 3, return_value=False)
    assert not val.any()


def test_li_mutation_is_detected():
    """A planted mistake in the oracle (ties broken by DESCENDING index) must be
    caught by the brute-force check -- shows the pinning has teeth."""
    sq = quantize(np.array([1.0, 2.0, 2.0, 2.0, 0.5], np.float32), "bf16")
    good, _ = LI.select_topk(sq, 5, 3)
    order = np.lexsort((-np.arange(5), -sq))   # mutated tie order
    bad = order[:3].astype(np.int32)
    want = _brute_topk(sq, 5, 3)
    assert np.array_equal(good, want) and not np.array_equal(bad, want)


def test_li_tnd_equals_per_batch_bsnd():
    lens_q, lens_k = [3, 5, 2], [4, 7, 2]
    N1, N2, D, K = 8, 1, 16, 4
    rng = np.random.RandomState(11)
    T1, T2 = sum(lens_q), sum(lens_k)
    q = round_bf16(rng.randn(T1, N1, D).astype(np.float32))
    k = round_bf16(rng.randn(T2, N2, D).astype(np.float32))
    w = rng.randn(T1, N1).astype(np.float32)
    cu_q, cu_k = np.cumsum(lens_q), np.cumsum(lens_k)
    idx, val = LI.lightning_indexer(q, k, w, cu_q, cu_k, layout_query="TND", layout_key="TND",
                                    sparse_count=K, sparse_mode=3, return_value=True)
    assert idx.shape == (T1, N2, K)
    oq = ok = 0
    for b in range(3):
        qb = q[oq:oq + lens_q[b]][None]
        kb = k[ok:ok + lens_k[b]][None]
        wb = w[oq:oq + lens_q[b]][None]
        ib, vb = LI.li_golden_bsnd(qb, kb, wb, [lens_q[b]], [lens_k[b]], K, 3, return_value=True)
        assert np.array_equal(idx[oq:oq + lens_q[b]], ib[0])
        assert np.array_equal(val[oq:oq + lens_q[b]], vb[0])
        oq += lens_q[b]
        ok += lens_k[b]


def test_parity_checker_accepts_midpoint_flip_only():
    # a value exactly at a bf16 midpoint may round either way; a far one may not
    s = np.array([1.00390625, 0.5, 0.25], np.float64)   # 1 + 2^-8: midpoint of 1 and 1+2^-7
    s32 = s.astype(np.float32)
    sq = quantize(s32, "bf16")
    stats = LiParityStats()
    flipped = np.array([1.0078125, 0.5, 0.25], np.float32)  # the other neighbour
    check_li_row(np.array([0, 1, 2], np.int32), flipped, s32, s, 3, 3, "bf16", stats)
    assert stats.flip_rows == 1
    with pytest.raises(AssertionError):
        wrong = np.array([1.0, 0.5, 0.2490234375], np.float32)  # 0.25 is exact: no flip allowed
        check_li_row(np.array([0, 1, 2], np.int32), wrong, s32, s, 3, 3, "bf16", stats)
    assert sq[0] == 1.0


# ----------------------------------------------------------------- SFA
def test_gather_positions_hand_cases():
    g = SFA.gather_positions
    # token-wise: scan limit = threshold, stops at the first -1
    assert g(np.array([0, 3, 5, -1, 2]), 1, 10, 10) == [0, 3, 5]
    assert g(np.array([0, 3, 5, 7]), 1, 2, 10) == [0]           # id 3 >= threshold 2 skipped
    assert g(np.array([0, 1, 1]), 1, 2, 10) == [0, 1]           # only ceil(2/1)=2 ids scanned
    assert g(np.array([9, 1]), 1, 5, 10) == [1]                 # id >= threshold skipped
    # block-wise bs=4: threshold 10 -> 3 ids scanned; clip to threshold
    assert g(np.array([2, 0, 1, 5]), 4, 10, 10) == [8, 9, 0, 1, 2, 3, 4, 5, 6, 7]
    # end clamped to act_k
    assert g(np.array([1]), 4, 8, 6) == [4, 5]
    assert g(np.array([-1, 0]), 2, 8, 8) == []
    assert g(np.array([0, 1]), 2, 3, 8) == [0, 1, 2]


def _sfa_tiny(B=1, S1=3, S2=9, N1=4, D=16, Dr=8, count=5, seed=0):
    rng = np.random.RandomState(seed)
    f = lambda *s: round_bf16(rng.randn(*s).astype(np.float32))
    return f(B, S1, N1, D), f(B, S2, 1, D), f(B, S1, N1, Dr), f(B, S2, 1, Dr)


@pytest.mark.parametrize("mode", [0, 3])
def test_sfa_golden_vs_float64_softmax(mode):
    B, S1, S2, N1, D, Dr, C = 2, 4, 12, 4, 16, 8, 6
    qn, kn, qr, kr = _sfa_tiny(B, S1, S2, N1, D, Dr, C, seed=1)
    rng = np.random.RandomState(2)
    si = np.full((B, S1, 1, C), -1, np.int32)
    for b in range(B):
        for s in range(S1):
            thr = S2 if mode == 0 else S2 - S1 + s + 1
            n = min(C, thr)
            si[b, s, 0, :n] = np.sort(rng.permutation(thr)[:n])
    scale = 1 / math.sqrt(D + Dr)
    out, smax, ssum = SFA.sfa_golden_bsnd(qn, kn, si, qr, kr, scale, [S1] * B, [S2] * B, 1, mode, "fp32")
    for b in range(B):
        for s in range(S1):
            pos = [int(x) for x in si[b, s, 0] if x >= 0]
            qf = torch.from_numpy(np.concatenate([qn[b, s], qr[b, s]], -1)).double()
            kf = torch.from_numpy(np.concatenate([kn[b, pos, 0], kr[b, pos, 0]], -1)).double()
            sc = qf @ kf.T * scale
            p = torch.softmax(sc, dim=-1)
            o = p @ torch.from_numpy(kn[b, pos, 0]).double()
            np.testing.assert_allclose(out[b, s], o.numpy(), rtol=1e-4, atol=1e-5)
            np.testing.assert_allclose(smax[b, 0, s], sc.max(-1).values.numpy(), rtol=1e-5, atol=1e-6)
            np.testing.assert_allclose(ssum[b, 0, s], torch.exp(sc - sc.max(-1, keepdim=True).values).sum(-1).numpy(), rtol=1e-5)
            assert np.all(ssum[b, 0, s] >= 1.0 - 1e-6)


def test_sfa_skip_rules():
    # mode 3 with act_q > act_k: leading rows s1 < aq - ak are zero
    qn, kn, qr, kr = _sfa_tiny(1, 6, 4, 2, 16, 8, 4, seed=3)
    si = np.tile(np.array([0, 1, 2, 3], np.int32), (1, 6, 1, 1))
    out, smax, ssum = SFA.sfa_golden_bsnd(qn, kn, si, qr, kr, 0.3, [6], [4], 1, 3, "bf16")
    assert not out[0, :2].any() and not smax[0, 0, :2].any() and not ssum[0, 0, :2].any()
    assert out[0, 2:].any()
    # row 2 sees threshold 1 -> only token 0: output == k[0] rounded, sm_sum == 1
    np.testing.assert_allclose(out[0, 2], np.broadcast_to(kn[0, 0, 0], (2, 16)), rtol=1e-2)
    assert np.allclose(ssum[0, 0, 2], 1.0)


def test_sfa_tnd_and_pa_equal_bsnd():
    rng = np.random.RandomState(4)
    N1, D, Dr, C, bs = 4, 16, 8, 5, 4
    lens_q, lens_k = [2, 3], [7, 10]
    T1, T2 = sum(lens_q), sum(lens_k)
    f = lambda *s: round_bf16(rng.randn(*s).astype(np.float32))
    q, qr = f(T1, N1, D), f(T1, N1, Dr)
    k, kr = f(T2, 1, D), f(T2, 1, Dr)
    si = np.full((T1, 1, C), -1, np.int32)
    r = 0
    for b in range(2):
        for s in range(lens_q[b]):
            thr = lens_k[b] - lens_q[b] + s + 1
            n = min(C, thr)
            si[r, 0, :n] = np.sort(rng.permutation(thr)[:n])
            r += 1
    scale = 0.25
    o_t, m_t, s_t = SFA.sparse_flash_attention(q, k, None, si, scale, None, np.cumsum(lens_q),
                                               np.cumsum(lens_k), qr, kr, 1, "TND", "TND", 3, True)
    assert o_t.shape == (T1, N1, D) and m_t.shape == (1, T1, N1)
    # PA: page the TND keys into blocks of 4 with a shuffled block table
    maxb = max((L + bs - 1) // bs for L in lens_k)
    nblk = sum((L + bs - 1) // bs for L in lens_k)
    perm = rng.permutation(nblk)
    cache = np.zeros((nblk, bs, 1, D), np.float32)
    cache_r = np.zeros((nblk, bs, 1, Dr), np.float32)
    bt = np.full((2, maxb), -1, np.int32)
    off = kb = 0
    for b in range(2):
        nb = (lens_k[b] + bs - 1) // bs
        for i in range(nb):
            blk = perm[kb]
            kb += 1
            bt[b, i] = blk
            seg = k[off + i * bs: off + min((i + 1) * bs, lens_k[b])]
            cache[blk, :seg.shape[0]] = seg
            cache_r[blk, :seg.shape[0]] = kr[off + i * bs: off + min((i + 1) * bs, lens_k[b])]
        off += lens_k[b]
    o_p, m_p, s_p = SFA.sparse_flash_attention(q, cache, None, si, scale, bt, np.cumsum(lens_q),
                                               lens_k, qr, cache_r, 1, "TND", "PA_BSND", 3, True,
                                               block_size=bs)
    assert np.array_equal(o_t, o_p) and np.array_equal(m_t, m_p) and np.array_equal(s_t, s_p)
    # per-batch BSND equivalence
    oq = ok = 0
    for b in range(2):
        ob, mb, sb = SFA.sfa_golden_bsnd(q[None, oq:oq + lens_q[b]], k[None, ok:ok + lens_k[b]],
                                         si[None, oq:oq + lens_q[b]], qr[None, oq:oq + lens_q[b]],
                                         kr[None, ok:ok + lens_k[b]], scale, [lens_q[b]], [lens_k[b]],
                                         1, 3, "bf16")
        assert np.array_equal(o_t[oq:oq + lens_q[b]], ob[0])
        assert np.array_equal(m_t[0, oq:oq + lens_q[b]], mb[0, 0])
        oq += lens_q[b]
        ok += lens_k[b]


# ----------------------------------------------------------------- workloads
def test_causal_index_generator_contract():
    from dsa_triton_ascend_amd.workloads import causal_block_indices, _gen
    for bs, mode in ((1, 3), (2, 3), (4, 0)):
        si = causal_block_indices(2, 16, 40, 8, bs, mode, _gen("cpu", 0), "cpu").numpy()
        for b in range(2):
            for s in range(16):
                thr = 40 if mode == 0 else 40 - 16 + s + 1
                nb = -(-thr // bs)
                row = si[b, s, 0]
                n = min(8, nb)
                assert np.all(row[n:] == -1)
                v = row[:n]
                assert np.all(np.diff(v) > 0) and v.min() >= 0 and v.max() < nb


@pytest.mark.parametrize("vd", ["bf16", "fp16"])
def test_parity_checker_accepts_other_fp32_order(vd):
    """An independent fp32 evaluation (d summed in 4 blocks, heads reversed) of the
    same scores must satisfy the parity rule -- the error bound covers real fp32
    reordering noise, including heavy cancellation with unscaled weights."""
    from tests.parity import check_li_row, row_error_bound
    rng = np.random.RandomState(21)
    S2, N1, D, K = 256, 64, 128, 64
    q = quantize(rng.randn(1, 24, N1, D).astype(np.float32), vd)
    k = quantize(rng.randn(1, S2, 1, D).astype(np.float32), vd)
    w = quantize(rng.randn(1, 24, N1).astype(np.float32), vd)
    stats = LiParityStats()
    for s1 in range(24):
        dots = np.zeros((S2, N1), np.float32)
        for blk in range(4):
            sl = slice(blk * 32, (blk + 1) * 32)
            dots += k[0, :, 0, sl] @ q[0, s1, :, sl].T
        alt = np.zeros(S2, np.float32)
        for g in reversed(range(N1)):
            alt += np.maximum(dots[:, g], 0) * w[0, s1, g]
        aq = quantize(alt, vd)
        gi, gv = LI.select_topk(aq, S2, K)
        s32 = LI.li_row_scores(q, k, w, 0, s1, 0, [24], [S2], 0)
        s64 = LI.li_row_scores_f64(q, k, w, 0, s1, 0, [24], [S2], 0)
        check_li_row(gi, gv, s32, s64, S2, K, vd, stats, err=row_error_bound(q, k, w, 0, s1, 0))
    assert stats.rows == 24


def test_parity_checker_rejects_dropped_head():
    """Planted mistake: scores missing one head's contribution must fail the rule."""
    from tests.parity import check_li_row, row_error_bound
    rng = np.random.RandomState(22)
    S2, N1, D, K = 128, 16, 64, 32
    q = round_bf16(rng.randn(1, 8, N1, D).astype(np.float32))
    k = round_bf16(rng.randn(1, S2, 1, D).astype(np.float32))
    w = (rng.randn(1, 8, N1) / 4).astype(np.float32)
    failures = 0
    for s1 in range(8):
        s32 = LI.li_row_scores(q, k, w, 0, s1, 0, [8], [S2], 0)
        wrong = s32 - np.maximum(k[0, :, 0] @ q[0, s1, 5], 0) * w[0, s1, 5]
        gi, gv = LI.select_topk(quantize(wrong, "bf16"), S2, K)
        s64 = LI.li_row_scores_f64(q, k, w, 0, s1, 0, [8], [S2], 0)
        try:
            check_li_row(gi, gv, s32, s64, S2, K, "bf16", LiParityStats(),
                         err=row_error_bound(q, k, w, 0, s1, 0))
        except AssertionError:
            failures += 1
    assert failures == 8


# ----------------------------------------------------------------- SFA backward
from oracle import sparse_flash_attention_grad_ref as SFG


def _autograd_sfa_grad(q, k, qr, kr, do, si, scale, act_q, act_k, bs, mode):
    """float64 torch autograd of the forward attention (value a separate leaf equal to
    k_nope, so d_key is the QK path only and d_value the PV path), plus the forward's
    exact output and softmax stats."""
    t = lambda x: torch.tensor(np.asarray(x, np.float64), requires_grad=True)
    tq, tk, tqr, tkr, tv = t(q), t(k), t(qr), t(kr), t(k)
    B, S1, N1, D = q.shape
    out = torch.zeros(B, S1, N1, D, dtype=torch.float64)
    smax = np.zeros((B, 1, S1, N1), np.float64)
    ssum = np.zeros((B, 1, S1, N1), np.float64)
    loss = torch.zeros((), dtype=torch.float64)
    for b in range(B):
        aq, ak = int(act_q[b]), int(act_k[b])
        for s1 in range(aq):
            if mode != 0 and s1 < aq - ak:
                continue
            thr = ak if mode == 0 else ak - aq + s1 + 1
            if thr <= 0:
                continue
            pos = SFA.gather_positions(si[b, s1, 0], bs, thr, ak)
            if not pos:
                continue
            pos = torch.tensor(pos)
            s = (tq[b, s1] @ tk[b, pos, 0].T + tqr[b, s1] @ tkr[b, pos, 0].T) * scale
            p = torch.softmax(s, dim=-1)
            o = p @ tv[b, pos, 0]
            loss = loss + (o * torch.from_numpy(np.asarray(do[b, s1], np.float64))).sum()
            out[b, s1] = o.detach()
            m = s.detach().max(dim=-1).values
            smax[b, 0, s1] = m.numpy()
            ssum[b, 0, s1] = torch.exp(s.detach() - m[:, None]).sum(-1).numpy()
    loss.backward()
    g = lambda x: x.grad.numpy() if x.grad is not None else np.zeros(x.shape)
    return out.numpy(), smax, ssum, (g(tq), g(tk), g(tv), g(tqr), g(tkr))


@pytest.mark.parametrize("mode,bs,act", [(3, 1, None), (0, 1, None), (3, 2, ([3, 2], [9, 6])),
                                         (0, 4, ([2, 3], [5, 12]))])
def test_sfa_grad_golden_vs_float64_autograd(mode, bs, act):
    """The backward golden (fed the forward's exact output and stats) equals float64
    autograd of the forward attention: catches a dropped delta, a misplaced scale, the
    d_key / d_value paths swapped or summed, and scatter-adds that lose duplicates."""
    B, S1, S2, N1, D, Dr = 2, 3, 12, 4, 16, 8
    rng = np.random.RandomState(5)
    q, qr, do = rng.randn(B, S1, N1, D), rng.randn(B, S1, N1, Dr), rng.randn(B, S1, N1, D)
    k, kr = rng.randn(B, S2, 1, D), rng.randn(B, S2, 1, Dr)
    act_q, act_k = act if act else ([S1] * B, [S2] * B)
    count = 5
    si = np.full((B, S1, 1, count), -1, np.int32)
    for b in range(B):
        for s1 in range(S1):
            nb = -(-S2 // bs)
            n = min(count, nb)
            si[b, s1, 0, :n] = np.sort(rng.permutation(nb)[:n])
    si[1, 2, 0, 3] = -1       # the scan of this row stops at its fourth id
    si[0, 2, 0, 1] = si[0, 2, 0, 0]   # a repeated id: the row gathers that position twice
    scale = 0.3
    out, smax, ssum, want = _autograd_sfa_grad(q, k, qr, kr, do, si, scale, act_q, act_k, bs, mode)
    got = SFG.sfa_grad_golden_bsnd(q, k, si, do, out, smax, ssum, qr, kr, scale, act_q, act_k,
                                   bs, mode, io_dtype="fp32")
    for name, gv, wv in zip(("dq", "dk", "dv", "dqr", "dkr"), got, want):
        np.testing.assert_allclose(gv, wv, rtol=2e-5, atol=2e-5, err_msg=name)
    # every token selected by several rows: the scatter must have summed them
    assert np.abs(want[2]).max() > 0


def test_sfa_grad_tnd_equals_bsnd():
    """TND wrapper == BSND golden on explicitly de-packed inputs (stats (1,T1,N1))."""
    rng = np.random.RandomState(6)
    lq, lk = [3, 2], [7, 5]
    T1, T2, N1, D, Dr = sum(lq), sum(lk), 2, 8, 4
    q, qr, do, o = (rng.randn(T1, N1, x).astype(np.float32) for x in (D, Dr, D, D))
    k, kr = rng.randn(T2, 1, D).astype(np.float32), rng.randn(T2, 1, Dr).astype(np.float32)
    sm, ss = rng.randn(1, T1, N1).astype(np.float32), (rng.rand(1, T1, N1) + 1).astype(np.float32)
    si = np.full((T1, 1, 4), -1, np.int32)
    for t in range(T1):
        b = 0 if t < lq[0] else 1
        si[t, 0, :3] = np.sort(rng.permutation(lk[b])[:3])
    cq, ck = np.cumsum(lq), np.cumsum(lk)
    got = SFG.sparse_flash_attention_grad(q, k, None, si, do, o, sm, ss, 0.5, qr, kr, cq, ck, 1, "TND", 3,
                                          io_dtype="fp32")
    ref_dq, ref_dqr = np.zeros_like(q), np.zeros_like(qr)
    ref_dk, ref_dv, ref_dkr = np.zeros_like(k), np.zeros_like(k), np.zeros_like(kr)
    q0 = k0 = 0
    for b in range(2):
        sl, kl = slice(q0, q0 + lq[b]), slice(k0, k0 + lk[b])
        r = SFG.sfa_grad_golden_bsnd(q[None, sl], k[None, kl], si[None, sl], do[None, sl], o[None, sl],
                                     sm[:, sl][None], ss[:, sl][None], qr[None, sl], kr[None, kl], 0.5,
                                     [lq[b]], [lk[b]], 1, 3, io_dtype="fp32")
        ref_dq[sl], ref_dk[kl], ref_dv[kl], ref_dqr[sl], ref_dkr[kl] = (x[0] for x in r)
        q0 += lq[b]
        k0 += lk[b]
    for gv, wv in zip(got, (ref_dq, ref_dk, ref_dv, ref_dqr, ref_dkr)):
        np.testing.assert_array_equal(gv, wv)


def test_li_pa_bsnd_equals_depaged_bsnd():
    """Paged keys (random block table, one -1 block) == the BSND golden on the de-paged
    keys built by hand: the -1 block's keys are zero rows (score 0, still selectable)."""
    rng = np.random.RandomState(8)
    B, S1, N1, D, page, mb = 2, 3, 8, 32, 4, 5
    q = round_bf16(rng.randn(B, S1, N1, D).astype(np.float32))
    w = rng.randn(B, S1, N1).astype(np.float32)
    nblk = 9
    cache = round_bf16(rng.randn(nblk, page, 1, D).astype(np.float32))
    bt = np.array([[3, 0, 7, -1, 5], [8, 1, 2, 4, 6]], np.int32)
    act_k = [18, 20]
    dense = np.zeros((B, mb * page, 1, D), np.float32)
    for b in range(B):
        for i in range(mb):
            if bt[b, i] >= 0:
                dense[b, i * page:(i + 1) * page] = cache[bt[b, i]]
    for mode in (0, 3):
        got = LI.lightning_indexer(q, cache, w, None, act_k, bt, "BSND", "PA_BSND", 6, mode, True)
        want = LI.lightning_indexer(q, dense, w, None, act_k, None, "BSND", "BSND", 6, mode, True)
        np.testing.assert_array_equal(got[0], want[0])
        np.testing.assert_array_equal(got[1], want[1])
    with pytest.raises(ValueError):
        LI.lightning_indexer(q, dense, w, block_table=bt)


# ----------------------------------------------------------------- sparse LI grad KL loss
from oracle import sli_grad_kl_loss_ref as SLI


def test_sli_grad_kl_loss_vs_float64_autograd():
    """Teacher p against torch.softmax over the full causal key range (averaged over
    heads, gathered at the slots); the loss against scipy's rel_entr; dW, dQI, dKI
    against float64 autograd of the surrogate -sum p log softmax(I) + (1 - sum p) lse(I),
    whose gradient in I is the golden's dI = softmax(I) - p. Repeated and out-of-range
    ids exercise the per-slot scatter and the clipping."""
    from scipy.special import rel_entr
    rng = np.random.RandomState(9)
    B, S1, S2, N1, D, Dr, G, Di, K = 2, 3, 16, 4, 8, 4, 3, 8, 6
    q, qr = rng.randn(B, S1, N1, D), rng.randn(B, S1, N1, Dr)
    k, kr = rng.randn(B, S2, 1, D), rng.randn(B, S2, 1, Dr)
    qi, ki, w = rng.randn(B, S1, G, Di), rng.randn(B, S2, 1, Di), np.abs(rng.randn(B, S1, G))
    si = rng.randint(0, S2, (B, S1, 1, K))
    si[0, 2, 0, 1] = si[0, 2, 0, 0]      # a repeated id
    si[1, 1, 0, 0] = S2 + 3              # clipped to S2 - 1
    scale = 0.4
    act_q, act_k = [S1, S1], [S2, 12]
    # full-row softmax stats over the causal range
    sm_max = np.zeros((B, 1, S1, N1))
    sm_sum = np.zeros((B, 1, S1, N1))
    for b in range(B):
        for s1 in range(S1):
            lim = act_k[b] - act_q[b] + s1 + 1
            sc = (q[b, s1] @ k[b, :lim, 0].T + qr[b, s1] @ kr[b, :lim, 0].T) * scale
            sm_max[b, 0, s1] = sc.max(1)
            sm_sum[b, 0, s1] = np.exp(sc - sc.max(1, keepdims=True)).sum(1)
    got = SLI.sli_grad_kl_loss(q, k, qr, kr, qi, ki, w, si, sm_max, sm_sum, scale, act_q, act_k, io_dtype="fp32")

    tqi, tki, tw = (torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in (qi, ki, w))
    total, loss_ref = 0.0, 0.0
    for b in range(B):
        for s1 in range(S1):
            lim = act_k[b] - act_q[b] + s1 + 1
            n = min(K, lim)
            idx = np.clip(si[b, s1, 0, :n], 0, S2 - 1)
            # teacher: the causal range's log-sum-exp normalises every key's probability
            # (a slot past the causal limit still gets exp(score - lse))
            sc = torch.tensor((q[b, s1] @ k[b, :, 0].T + qr[b, s1] @ kr[b, :, 0].T) * scale)
            lse = torch.logsumexp(sc[:, :lim], dim=-1, keepdim=True)
            p = torch.exp(sc - lse).mean(0)[torch.tensor(idx)]
            ii = (torch.relu(tqi[b, s1] @ tki[b, torch.tensor(idx), 0].T) * tw[b, s1][:, None]).sum(0)
            lsm = torch.log_softmax(ii, dim=0)
            total = total - (p * lsm).sum() + (1 - p.sum()) * torch.logsumexp(ii, 0)
            loss_ref += float(rel_entr(np.maximum(p.numpy(), 1e-8), np.maximum(torch.exp(lsm).detach().numpy(), 1e-8)).sum())
    total.backward()
    np.testing.assert_allclose(got[0], tqi.grad.numpy(), rtol=1e-4, atol=1e-5, err_msg="dQI")
    np.testing.assert_allclose(got[1], tki.grad.numpy(), rtol=1e-4, atol=1e-5, err_msg="dKI")
    np.testing.assert_allclose(got[2], tw.grad.numpy(), rtol=1e-4, atol=1e-5, err_msg="dW")
    np.testing.assert_allclose(got[3][0], loss_ref, rtol=1e-4)


# ----------------------------------------------------------------- dense indexer loss
from oracle import dense_loss_ref as DLO


def test_dense_lse_vs_scipy_logsumexp():
    from scipy.special import logsumexp
    rng = np.random.RandomState(10)
    B, S1, S2, G, Di = 2, 4, 9, 3, 8
    qi, ki, w = rng.randn(B, S1, G, Di), rng.randn(B, S2, 1, Di), np.abs(rng.randn(B, S1, G))
    act_q, act_k = [4, 3], [9, 5]
    mx, sm = DLO.dense_softmax_lse(qi, ki, w, act_q, act_k)
    for b in range(B):
        for s1 in range(S1):
            n = min(max(act_k[b] - act_q[b] + s1 + 1, 0), act_k[b], S2) if s1 < act_q[b] else 0
            if n == 0:
                assert mx[b, 0, s1] == -np.inf and sm[b, 0, s1] == 0
                continue
            ii = (np.maximum(qi[b, s1] @ ki[b, :n, 0].T, 0) * w[b, s1][:, None]).sum(0)
            np.testing.assert_allclose(np.log(sm[b, 0, s1]) + mx[b, 0, s1], logsumexp(ii), rtol=1e-5)


def test_dense_loss_equals_sparse_loss_over_all_visible_keys():
    """With one KV head (N2 = 1) the dense loss is the sparse one whose slots are all the
    visible keys in order (the two differ only by the 1e-8 placement in the indexer
    softmax); with N2 = N1 the teacher of each head reads its own key head, checked
    against per-head torch softmax over the causal range."""
    rng = np.random.RandomState(11)
    B, S1, S2, N1, D, G, Di = 1, 3, 10, 4, 8, 2, 8
    q, qr, k, kr = rng.randn(B, S1, N1, D), rng.randn(B, S1, N1, 4), rng.randn(B, S2, 1, D), rng.randn(B, S2, 1, 4)
    qi, ki, w = rng.randn(B, S1, G, Di), rng.randn(B, S2, 1, Di), np.abs(rng.randn(B, S1, G))
    scale = 0.3
    sm_max, sm_sum = np.zeros((B, 1, S1, N1)), np.zeros((B, 1, S1, N1))
    for s1 in range(S1):
        lim = S2 - S1 + s1 + 1
        sc = (q[0, s1] @ k[0, :lim, 0].T + qr[0, s1] @ kr[0, :lim, 0].T) * scale
        sm_max[0, 0, s1] = sc.max(1)
        sm_sum[0, 0, s1] = np.exp(sc - sc.max(1, keepdims=True)).sum(1)
    mxi, smi = DLO.dense_softmax_lse(qi, ki, w)
    got = DLO.dense_loss_backward(q, k, qr, kr, qi, ki, w, sm_max, sm_sum, mxi, smi, scale, io_dtype="fp32")
    si = np.tile(np.arange(S2, dtype=np.int32), (B, S1, 1, 1))
    want = SLI.sli_grad_kl_loss(q, k, qr, kr, qi, ki, w, si, sm_max, sm_sum, scale, io_dtype="fp32")
    for gv, wv in zip(got, want):
        np.testing.assert_allclose(gv, wv, rtol=1e-5, atol=1e-7)
    # grouped heads: N2 = N1, stats [B, N2, S1, 1]
    k2, kr2 = rng.randn(B, S2, N1, D), rng.randn(B, S2, N1, 4)
    sm2, ss2 = np.zeros((B, N1, S1, 1)), np.zeros((B, N1, S1, 1))
    p_ref = []
    for s1 in range(S1):
        lim = S2 - S1 + s1 + 1
        sc = np.stack([(q[0, s1, h] @ k2[0, :lim, h].T + qr[0, s1, h] @ kr2[0, :lim, h].T) * scale for h in range(N1)])
        sm2[0, :, s1, 0] = sc.max(1)
        ss2[0, :, s1, 0] = np.exp(sc - sc.max(1, keepdims=True)).sum(1)
        p_ref.append(torch.softmax(torch.tensor(sc), -1).mean(0).numpy())
    got2 = DLO.dense_loss_backward(q, k2, qr, kr2, qi, ki, w, sm2, ss2, mxi, smi, scale, io_dtype="fp32")
    # the teacher enters the loss: recompute it from p_ref and the student of the same rows
    loss = 0.0
    for s1 in range(S1):
        n = S2 - S1 + s1 + 1
        ii = (np.maximum(qi[0, s1] @ ki[0, :n, 0].T, 0) * w[0, s1][:, None]).sum(0)
        st = np.exp(ii - mxi[0, 0, s1]) / smi[0, 0, s1]
        p = np.maximum(p_ref[s1], 1e-8)
        loss += float(np.sum(p * (np.log(p) - np.log(np.maximum(st, 1e-8)))))
    np.testing.assert_allclose(got2[3][0], loss, rtol=1e-5)
