"""GPU parity: sparse_flash_attention (HIP) vs the oracle
(oracle/sparse_flash_attention_ref.py).

Shape matrix follows the reference's test_golden (test_sfa_triton.py:129-169):
token-wise and block-wise (bs 2, 4), S1=1, topK=2048, multi-batch,
D in {128,256,512}, fp16 / bf16, plus mode 0, TND and PA_BSND cases the
reference never tests. Tolerances: outputs within rtol=atol=1e-2 (io dtype),
softmax_max / softmax_sum within rtol 1e-4 (fp32).
"""
import math

import numpy as np
import pytest
import torch

from dsa_triton_ascend_amd import SparseFlashAttention, sparse_flash_attention
from dsa_triton_ascend_amd import workloads as W
from oracle import sparse_flash_attention_ref as SFA

pytestmark = pytest.mark.gpu

DT = {"bf16": torch.bfloat16, "fp16": torch.float16}
OUT_TOL = dict(rtol=1e-2, atol=1e-2)
LSE_TOL = dict(rtol=1e-4, atol=1e-5)


def _np(t):
    return t.float().cpu().numpy()


def _ref_indices(B, S1, S2, count, bs, mode, seed=7):
    """Reference index generator (test_sfa_triton.py:64-85), same RandomState(7) stream."""
    rng = np.random.RandomState(seed)
    si = np.full((B, S1, 1, count), -1, dtype=np.int32)
    for b in range(B):
        for s1 in range(S1):
            thr = S2 if mode == 0 else S2 - S1 + s1 + 1
            if thr <= 0:
                continue
            nb = int(np.ceil(thr / bs))
            n = min(count, nb)
            si[b, s1, 0, :n] = np.sort(rng.permutation(nb)[:n]).astype(np.int32)
    return si


def _inputs(B, S1, S2, N1, D, dtype, seed=42):
    """Reference generator semantics (test_sfa_triton.py:47-61): randn -> fp16 -> dtype."""
    rng = np.random.RandomState(seed)
    t = lambda *s: torch.from_numpy(rng.randn(*s).astype(np.float16)).to(DT[dtype])
    q, k, v, qr, kr = t(B, S1, N1, D), t(B, S2, 1, D), t(B, S2, 1, D), t(B, S1, N1, 64), t(B, S2, 1, 64)
    return q, k, v, qr, kr


ROW_REL_TOL = 1e-2   # per (row, head): ||out - oracle|| / ||oracle|| over the D columns


def row_rel_err(go, o_out):
    """Per (row, head) relative L2 error of the output rows. Rows the oracle leaves at
    zero (skipped rows, rows without tokens) must be exactly zero. Elementwise 1e-2
    tolerances alone would pass a 30% error on outputs of magnitude ~0.03 (long rows
    average thousands of value rows); this bound would not."""
    d = go.reshape(-1, go.shape[-1]).astype(np.float64)
    r = o_out.reshape(-1, o_out.shape[-1]).astype(np.float64)
    nr = np.linalg.norm(r, axis=1)
    nd = np.linalg.norm(d - r, axis=1)
    zero = nr == 0
    assert np.all(nd[zero] == 0), "rows the oracle leaves at zero are not zero"
    return float((nd[~zero] / nr[~zero]).max()) if (~zero).any() else 0.0


def compare(out, smax, ssum, o_out, o_max, o_sum, what):
    go, gm, gs = _np(out), _np(smax), _np(ssum)
    assert go.shape == o_out.shape and gm.shape == o_max.shape
    assert np.all(np.isfinite(go))
    np.testing.assert_allclose(go, o_out, err_msg=f"{what}: attention_out", **OUT_TOL)
    np.testing.assert_allclose(gm, o_max, err_msg=f"{what}: softmax_max", **LSE_TOL)
    np.testing.assert_allclose(gs, o_sum, err_msg=f"{what}: softmax_sum", **LSE_TOL)
    rel = row_rel_err(go, o_out)
    assert rel <= ROW_REL_TOL, f"{what}: per-row relative error {rel:.3e} > {ROW_REL_TOL}"
    err = np.abs(go - o_out).max()
    print(f"[sfa parity] {what}: max|out-oracle|={err:.3e} max row rel={rel:.2e} "
          f"max|lse rel|={np.max(np.abs(gs - o_sum) / np.maximum(np.abs(o_sum), 1e-30)):.2e}")


GOLDEN = [(1, 4, 128, 8, 64, 1, 3), (2, 16, 256, 16, 128, 1, 3), (1, 8, 128, 8, 32, 2, 3),
          (1, 8, 256, 16, 32, 4, 3), (1, 1, 128, 8, 16, 1, 3), (1, 4, 2048, 8, 2048, 1, 3),
          (1, 4, 128, 8, 64, 1, 0), (1, 4, 2048, 8, 2048, 1, 0)]


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("D", [128, 256, 512])
@pytest.mark.parametrize("B,S1,S2,N1,count,bs,mode", GOLDEN)
def test_golden_matrix(dev, B, S1, S2, N1, count, bs, mode, D, dtype):
    q, k, v, qr, kr = _inputs(B, S1, S2, N1, D, dtype)
    si = _ref_indices(B, S1, S2, count, bs, mode)
    scale = 1.0 / math.sqrt(D + 64)
    mod = SparseFlashAttention(scale_value=scale, sparse_block_size=bs, sparse_mode=mode,
                               return_softmax_lse=True)
    out, smax, ssum = mod(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(si).to(dev),
                          query_rope=qr.to(dev), key_rope=kr.to(dev))
    torch.cuda.synchronize()
    o = SFA.sparse_flash_attention(_np(q), _np(k), None, si, scale, query_rope=_np(qr),
                                   key_rope=_np(kr), sparse_block_size=bs, sparse_mode=mode,
                                   return_softmax_lse=True, io_dtype=dtype)
    assert out.dtype == q.dtype and smax.shape == (B, 1, S1, N1)
    compare(out, smax, ssum, *o, what=f"B{B} S1={S1} S2={S2} N1={N1} k={count} bs={bs} m{mode} D{D} {dtype}")


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("D", [128, 256])
@pytest.mark.parametrize("S1,S2,count", [(6, 300, 200), (1, 2100, 2048)])
def test_per_wave_pv_form_smaller_d(dev, S1, S2, count, D, dtype):
    """128 heads at D = 128 / 256: the per-wave PV form with its Q^T staged through the gather
    ring at those row widths (two or four heads per copy instruction), on unsplit rows with a
    partial last tile and on a single decode-like row that is split over KV."""
    B, N1 = 1, 128
    q, k, v, qr, kr = _inputs(B, S1, S2, N1, D, dtype, seed=21)
    si = _ref_indices(B, S1, S2, count, 1, 3, seed=22)
    scale = 1.0 / math.sqrt(D + 64)
    out, smax, ssum = sparse_flash_attention(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(si).to(dev),
                                             scale_value=scale, query_rope=qr.to(dev), key_rope=kr.to(dev),
                                             sparse_mode=3, return_softmax_lse=True)
    o = SFA.sparse_flash_attention(_np(q), _np(k), None, si, scale, query_rope=_np(qr), key_rope=_np(kr),
                                   sparse_mode=3, return_softmax_lse=True, io_dtype=dtype)
    compare(out, smax, ssum, *o, what=f"N1=128 D={D} S1={S1} S2={S2} k={count} {dtype}")


@pytest.mark.parametrize("N1", [1, 2, 32, 64, 128])
def test_head_counts(dev, N1):
    B, S1, S2, D, count = 1, 6, 96, 512, 48
    q, k, v, qr, kr = _inputs(B, S1, S2, N1, D, "bf16", seed=5)
    si = _ref_indices(B, S1, S2, count, 1, 3, seed=8)
    out, smax, ssum = sparse_flash_attention(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(si).to(dev),
                                             scale_value=0.05, query_rope=qr.to(dev), key_rope=kr.to(dev),
                                             sparse_mode=3, return_softmax_lse=True)
    o = SFA.sparse_flash_attention(_np(q), _np(k), None, si, 0.05, query_rope=_np(qr), key_rope=_np(kr),
                                   sparse_mode=3, return_softmax_lse=True, io_dtype="bf16")
    compare(out, smax, ssum, *o, what=f"N1={N1}")


@pytest.mark.parametrize("scale", [-0.05, 0.0])
@pytest.mark.parametrize("N1", [16, 128])
def test_non_positive_scale(dev, N1, scale):
    """The softmax runs on raw scores times a positive scale: a negative scale_value
    runs on the negated query, zero as 1e-30. Both must match the oracle (zero: every
    valid token weighs the same, softmax_max 0), including partial last tiles."""
    B, S1, S2, D, count = 1, 5, 100, 512, 70
    q, k, v, qr, kr = _inputs(B, S1, S2, N1, D, "bf16", seed=6)
    si = _ref_indices(B, S1, S2, count, 1, 3, seed=9)
    out, smax, ssum = sparse_flash_attention(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(si).to(dev),
                                             scale_value=scale, query_rope=qr.to(dev), key_rope=kr.to(dev),
                                             sparse_mode=3, return_softmax_lse=True)
    o = SFA.sparse_flash_attention(_np(q), _np(k), None, si, scale, query_rope=_np(qr), key_rope=_np(kr),
                                   sparse_mode=3, return_softmax_lse=True, io_dtype="bf16")
    compare(out, smax, ssum, *o, what=f"N1={N1} scale={scale}")


def test_actual_lengths_and_skips(dev):
    """act_q > act_k (mode-3 leading rows skipped), a -1 in the middle of a row
    (scan stops), duplicate ids, ids beyond the threshold."""
    B, S1, S2, N1, D, count = 2, 8, 64, 16, 128, 12
    q, k, v, qr, kr = _inputs(B, S1, S2, N1, D, "bf16", seed=9)
    rng = np.random.RandomState(1)
    si = rng.randint(0, 64, size=(B, S1, 1, count)).astype(np.int32)
    si[0, 3, 0, 5] = -1
    si[1, 2, 0, :] = 7
    act_q, act_k = [8, 6], [5, 64]
    for mode in (0, 3):
        out, smax, ssum = sparse_flash_attention(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(si).to(dev),
                                                 scale_value=0.07, actual_seq_lengths_query=act_q,
                                                 actual_seq_lengths_kv=act_k, query_rope=qr.to(dev),
                                                 key_rope=kr.to(dev), sparse_mode=mode,
                                                 return_softmax_lse=True)
        o = SFA.sparse_flash_attention(_np(q), _np(k), None, si, 0.07, None, act_q, act_k, _np(qr),
                                       _np(kr), 1, "BSND", "BSND", mode, True, io_dtype="bf16")
        compare(out, smax, ssum, *o, what=f"act lengths mode {mode}")


def test_lse_not_requested_gives_zeros(dev):
    q, k, v, qr, kr = _inputs(1, 4, 64, 8, 128, "bf16")
    si = _ref_indices(1, 4, 64, 16, 1, 3)
    out, smax, ssum = sparse_flash_attention(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(si).to(dev),
                                             scale_value=0.1, query_rope=qr.to(dev), key_rope=kr.to(dev),
                                             sparse_mode=3, return_softmax_lse=False)
    assert not smax.any() and not ssum.any() and out.abs().sum() > 0


def test_tnd(dev):
    lens_q, lens_k = [5, 1, 40, 17], [64, 9, 40, 100]
    N1, D, count = 16, 512, 32
    rng = np.random.RandomState(2)
    T1, T2 = sum(lens_q), sum(lens_k)
    f = lambda *s: torch.from_numpy(rng.randn(*s).astype(np.float32)).bfloat16()
    q, qr, k, kr = f(T1, N1, D), f(T1, N1, 64), f(T2, 1, D), f(T2, 1, 64)
    si = np.full((T1, 1, count), -1, np.int32)
    r = 0
    for b in range(4):
        for s in range(lens_q[b]):
            thr = lens_k[b] - lens_q[b] + s + 1
            if thr > 0:
                n = min(count, thr)
                si[r, 0, :n] = np.sort(rng.permutation(thr)[:n])
            r += 1
    cq, ck = np.cumsum(lens_q).tolist(), np.cumsum(lens_k).tolist()
    out, smax, ssum = sparse_flash_attention(q.to(dev), k.to(dev), k.to(dev), torch.from_numpy(si).to(dev),
                                             scale_value=0.04, actual_seq_lengths_query=cq,
                                             actual_seq_lengths_kv=ck, query_rope=qr.to(dev),
                                             key_rope=kr.to(dev), layout_query="TND", layout_kv="TND",
                                             sparse_mode=3, return_softmax_lse=True)
    assert out.shape == (T1, N1, D) and smax.shape == (1, T1, N1)
    o = SFA.sparse_flash_attention(_np(q), _np(k), None, si, 0.04, None, cq, ck, _np(qr), _np(kr), 1,
                                   "TND", "TND", 3, True, io_dtype="bf16")
    compare(out, smax, ssum, *o, what="TND")


def test_pa_decode_small(dev):
    """PA_BSND decode with a shuffled block table and a -1 (missing) block."""
    inp = W.sfa_decode_inputs(B=4, N1=128, len_lo=300, len_hi=700, block_size=64, sparse_count=128,
                              device="cpu", seed=3)
    bt = inp.block_table.clone()
    bt[1, 2] = -1   # tokens of this block read as zeros, like the reference's de-paging
    out, smax, ssum = sparse_flash_attention(inp.query.to(dev), inp.key.to(dev), inp.key.to(dev),
                                             inp.sparse_indices.to(dev), scale_value=inp.scale_value,
                                             block_table=bt.to(dev),
                                             actual_seq_lengths_kv=inp.actual_seq_lengths_kv,
                                             query_rope=inp.query_rope.to(dev), key_rope=inp.key_rope.to(dev),
                                             layout_kv="PA_BSND", sparse_mode=3, return_softmax_lse=True,
                                             block_size=64)
    o = SFA.sparse_flash_attention(_np(inp.query), _np(inp.key), None, inp.sparse_indices.numpy(),
                                   inp.scale_value, bt.numpy(), None, inp.actual_seq_lengths_kv,
                                   _np(inp.query_rope), _np(inp.key_rope), 1, "BSND", "PA_BSND", 3, True,
                                   block_size=64, io_dtype="bf16")
    compare(out, smax, ssum, *o, what="PA decode small")


def test_c4_decode_full(dev):
    """BASELINE config 4 at full size; the oracle runs every one of the 64 rows (in four
    groups of 16 batches, so its de-paged key copy stays ~1.2 GB)."""
    inp = W.sfa_decode_inputs(device=dev, seed=42)
    out, smax, ssum = sparse_flash_attention(inp.query, inp.key, inp.key, inp.sparse_indices,
                                             **inp.kwargs())
    torch.cuda.synchronize()
    kc, krc = _np(inp.key), _np(inp.key_rope)
    for g0 in range(0, 64, 16):
        sel = list(range(g0, g0 + 16))
        o = SFA.sparse_flash_attention(_np(inp.query[sel]), kc, None,
                                       inp.sparse_indices[sel].cpu().numpy(), inp.scale_value,
                                       inp.block_table[sel].cpu().numpy(), None,
                                       [inp.actual_seq_lengths_kv[b] for b in sel], _np(inp.query_rope[sel]),
                                       krc, 1, "BSND", "PA_BSND", 3, True,
                                       block_size=inp.block_size, io_dtype="bf16")
        compare(out[sel], smax[sel], ssum[sel], *o, what=f"C4 decode (batches {g0}..{g0 + 15})")


def _climbing_inputs(S1, N1, D, dtype, climbs, seed=0):
    """Keys whose score against every head climbs from tile to tile: key rows are small
    noise except one spike per 32-token tile, k_t = a_j * u with u a fixed +-1 vector, and
    query rows u * c_r + noise/2 (c_r = 1, 0.8, 1.2, -1), so the spike of tile j scores
    about c_r * level_j with level_j climbing by `climbs` nats per tile (15-35). Tile 7 gets
    a second spike 0.5 nats below its first, so the output mixes two value rows."""
    rng = np.random.RandomState(seed)
    S2 = 256
    scale = 1.0 / math.sqrt(D + 64)
    u = np.where(rng.rand(D) < 0.5, -1.0, 1.0).astype(np.float32)
    k = (0.05 * rng.randn(S2, D)).astype(np.float32)
    level = 0.0
    for j in range(1, S2 // 32):
        level += climbs[(j - 1) % len(climbs)]
        k[j * 32 + rng.randint(31)] = level / (D * scale) * u          # positions 0..30 of the tile
    k[S2 - 1] = (level - 0.5) / (D * scale) * u                         # second spike of the last tile
    c = np.array([1.0, 0.8, 1.2, -1.0] * ((S1 + 3) // 4))[:S1]
    q = c[:, None, None] * u[None, None, :] + 0.5 * rng.randn(S1, N1, D)
    qr = 0.5 * rng.randn(S1, N1, 64)
    kr = 0.05 * rng.randn(S2, 64)
    t = lambda x: torch.from_numpy(np.asarray(x, np.float32)).to(DT[dtype])
    return (t(q[None]), t(k[None, :, None]), t(qr[None]), t(kr[None, :, None]), scale)


@pytest.mark.parametrize("N1", [32, 128])
@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("D", [128, 512])
@pytest.mark.parametrize("climbs", [(15.0,), (35.0, 15.0, 22.0)])
def test_climbing_score_spread(dev, dtype, D, climbs, N1):
    """Rows whose per-tile score maxima climb by 15-35 nats (total spread ~100-180 nats):
    with the exponent reference held back by the lazy-rescale threshold, P = exp(s - m_used)
    reaches e^TAU before it is packed to the io dtype. Outputs must stay finite and match
    the oracle, unsplit (one work-group per row) and over forced KV splits (each split
    listing its own tokens and a merge)."""
    S1 = 4
    q, k, qr, kr, scale = _climbing_inputs(S1, N1, D, dtype, climbs)
    si = np.tile(np.arange(256, dtype=np.int32), (1, S1, 1, 1))
    o = SFA.sparse_flash_attention(_np(q), _np(k), None, si, scale, query_rope=_np(qr), key_rope=_np(kr),
                                   sparse_mode=0, return_softmax_lse=True, io_dtype=dtype)
    assert o[1].max() > 100   # the spread is there
    for kv_splits in (1, 4):
        out, smax, ssum = sparse_flash_attention(q.to(dev), k.to(dev), k.to(dev), torch.from_numpy(si).to(dev),
                                                 scale_value=scale, query_rope=qr.to(dev), key_rope=kr.to(dev),
                                                 sparse_mode=0, return_softmax_lse=True, kv_splits=kv_splits)
        torch.cuda.synchronize()
        compare(out, smax, ssum, *o, what=f"climbing {climbs} D{D} {dtype} kv_splits={kv_splits}")


@pytest.mark.slow
def test_c3_prefill_sampled(dev):
    """BASELINE config 3 at full size; oracle on stride-sampled rows."""
    inp = W.sfa_prefill_inputs(device=dev, seed=42)
    out, smax, ssum = sparse_flash_attention(inp.query, inp.key, inp.key, inp.sparse_indices,
                                             **inp.kwargs())
    torch.cuda.synchronize()
    # 128 stride-sampled rows over the whole causal triangle plus its corners
    rows = [(0, s) for s in sorted(set(range(5, 4096, 32)) | {0, 1, 2047, 2048, 4095})]
    assert len(rows) >= 128
    o = SFA.sparse_flash_attention(_np(inp.query), _np(inp.key), None, inp.sparse_indices.cpu().numpy(),
                                   inp.scale_value, query_rope=_np(inp.query_rope), key_rope=_np(inp.key_rope),
                                   sparse_mode=3, return_softmax_lse=True, io_dtype="bf16", rows=rows)
    s = [r[1] for r in rows]
    compare(out[:, s], smax[:, :, s], ssum[:, :, s], o[0][:, s], o[1][:, :, s], o[2][:, :, s],
            what="C3 prefill (sampled rows)")


@pytest.mark.slow
@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_perf_sfa_shape_forward(dev, dtype):
    """The reference's perf_sfa shape (perf_sfa_triton.py:7-9: B=1, S1=512, S2=4096, N1=64,
    top-k 2048, D=512+64, causal) -- the bench's sfa_prefill_n64 line: every one of the 512
    rows against the oracle. Rows near the end select 2048 tokens (64 tiles), so the
    64-head forward's lazy rescaling runs over full-length rows."""
    inp = W.sfa_prefill_inputs(B=1, S1=512, S2=4096, N1=64, D=512, sparse_count=2048, device=dev,
                               seed=42, dtype=DT[dtype])
    out, smax, ssum = sparse_flash_attention(inp.query, inp.key, inp.key, inp.sparse_indices,
                                             **inp.kwargs())
    torch.cuda.synchronize()
    o = SFA.sparse_flash_attention(_np(inp.query), _np(inp.key), None, inp.sparse_indices.cpu().numpy(),
                                   inp.scale_value, query_rope=_np(inp.query_rope), key_rope=_np(inp.key_rope),
                                   sparse_mode=3, return_softmax_lse=True, io_dtype=dtype)
    compare(out, smax, ssum, *o, what=f"perf_sfa shape N1=64 {dtype} (all 512 rows)")


@pytest.mark.parametrize("N1,dtype,mode", [(128, "bf16", 3), (128, "fp16", 3), (128, "bf16", 0)])
def test_rows_mixed_lengths(dev, N1, dtype, mode):
    """2 x 700 unsplit rows of 128 heads at D = 512 (more rows than CUs) whose token
    counts vary from 0 to 8 tiles: ids cut short by a -1 at a random position (rows
    without tokens among rows with tokens), partial last tiles. Every row is checked
    against the oracle."""
    B, S1, S2, D, count = 2, 700, 900, 512, 256
    q, k, v, qr, kr = _inputs(B, S1, S2, N1, D, dtype, seed=11)
    si = _ref_indices(B, S1, S2, count, 1, mode, seed=12)
    rng = np.random.RandomState(13)
    cut = rng.randint(0, count + 1, size=(B, S1))
    cut[rng.rand(B, S1) < 0.4] = count   # most rows keep every id
    for b in range(B):
        for s in range(S1):
            si[b, s, 0, cut[b, s]:] = -1
    out, smax, ssum = sparse_flash_attention(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(si).to(dev),
                                             scale_value=0.04, query_rope=qr.to(dev), key_rope=kr.to(dev),
                                             sparse_mode=mode, return_softmax_lse=True)
    torch.cuda.synchronize()
    o = SFA.sparse_flash_attention(_np(q), _np(k), None, si, 0.04, query_rope=_np(qr), key_rope=_np(kr),
                                   sparse_mode=mode, return_softmax_lse=True, io_dtype=dtype)
    compare(out, smax, ssum, *o, what=f"mixed rows N1={N1} {dtype} m{mode}")


def test_pa_many_rows_token_list(dev):
    """PA_BSND with 1,088 query rows, so the one-wave-per-row token-list kernel runs with a
    block table: shuffled pages, a missing (-1) page, a -1 in the middle of a row (the scan
    stops there), -1 tail padding and rows shorter than the count."""
    B = 1088
    inp = W.sfa_decode_inputs(B=B, N1=8, len_lo=40, len_hi=400, block_size=32, sparse_count=48,
                              device="cpu", seed=11)
    si = inp.sparse_indices.clone()
    si[5, 0, 0, 7] = -1           # stop mid-row
    si[1024, 0, 0, 20:] = -1      # tail padding
    bt = inp.block_table.clone()
    bt[9, 1] = -1                 # a missing page reads as zeros
    out, smax, ssum = sparse_flash_attention(inp.query.to(dev), inp.key.to(dev), inp.key.to(dev),
                                             si.to(dev), scale_value=inp.scale_value, block_table=bt.to(dev),
                                             actual_seq_lengths_kv=inp.actual_seq_lengths_kv,
                                             query_rope=inp.query_rope.to(dev), key_rope=inp.key_rope.to(dev),
                                             layout_kv="PA_BSND", sparse_mode=3, return_softmax_lse=True,
                                             block_size=32)
    torch.cuda.synchronize()
    sel = [0, 5, 9, 1023, 1024, 1087] + list(range(13, B, 97))
    o = SFA.sparse_flash_attention(_np(inp.query[sel]), _np(inp.key), None, si[sel].numpy(),
                                   inp.scale_value, bt[sel].numpy(), None,
                                   [inp.actual_seq_lengths_kv[b] for b in sel], _np(inp.query_rope[sel]),
                                   _np(inp.key_rope), 1, "BSND", "PA_BSND", 3, True,
                                   block_size=32, io_dtype="bf16")
    compare(out[sel], smax[sel], ssum[sel], *o, what="PA 1088 rows (token list per wave)")


@pytest.mark.parametrize("kv_splits", [2, 5, 16])
def test_forced_kv_splits_with_empty_splits(dev, kv_splits):
    """Forced KV splits on short rows: splits past a row's token list are empty (they store
    zeros and l = 0); the merge must weight them out. Also rows with no tokens at all."""
    B, S1, S2, N1, D, count = 1, 6, 96, 16, 512, 96
    q, k, v, qr, kr = _inputs(B, S1, S2, N1, D, "bf16", seed=21)
    si = _ref_indices(B, S1, S2, count, 1, 3, seed=5)
    out, smax, ssum = sparse_flash_attention(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(si).to(dev),
                                             scale_value=0.05, query_rope=qr.to(dev), key_rope=kr.to(dev),
                                             sparse_mode=3, return_softmax_lse=True, kv_splits=kv_splits)
    o = SFA.sparse_flash_attention(_np(q), _np(k), None, si, 0.05, None, None, None, _np(qr), _np(kr), 1,
                                   "BSND", "BSND", 3, True, io_dtype="bf16")
    compare(out, smax, ssum, *o, what=f"kv_splits={kv_splits}")


@pytest.mark.parametrize("N1", [16, 64, 128])
@pytest.mark.parametrize("kv_splits", [2, 5])
def test_forced_kv_splits_block_size_2(dev, N1, kv_splits):
    """KV splits over token lists built by the token-list launch (sparse_block_size 2): at
    D = 512 the 8-wave attention forms (N1 <= 64, and N1 = 128) write the split
    partials and the merge combines them, including splits past a short row's tokens."""
    B, S1, S2, D, count, bs = 1, 8, 160, 512, 48, 2
    q, k, v, qr, kr = _inputs(B, S1, S2, N1, D, "bf16", seed=23)
    si = _ref_indices(B, S1, S2, count, bs, 3, seed=6)
    out, smax, ssum = sparse_flash_attention(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(si).to(dev),
                                             scale_value=0.05, query_rope=qr.to(dev), key_rope=kr.to(dev),
                                             sparse_block_size=bs, sparse_mode=3, return_softmax_lse=True,
                                             kv_splits=kv_splits)
    o = SFA.sparse_flash_attention(_np(q), _np(k), None, si, 0.05, None, None, None, _np(qr), _np(kr), bs,
                                   "BSND", "BSND", 3, True, io_dtype="bf16")
    compare(out, smax, ssum, *o, what=f"N1={N1} bs={bs} kv_splits={kv_splits}")


@pytest.mark.parametrize("mode", [0, 3])
def test_split_token_lists_long_scan(dev, mode):
    """KV-split rows that list their own tokens when the scan spans several 2048-id
    passes (sparse_count 5000): a -1 in the third pass stops one row, another row's
    scan ends at its threshold, ids past act_k are skipped; default and forced splits."""
    B, S1, S2, N1, D, count = 1, 3, 6000, 8, 128, 5000
    q, k, v, qr, kr = _inputs(B, S1, S2, N1, D, "bf16", seed=31)
    rng = np.random.RandomState(3)
    si = np.stack([np.sort(rng.permutation(S2)[:count]) for _ in range(S1)]).astype(np.int32)
    si = si.reshape(B, S1, 1, count)
    si[0, 1, 0, 4500] = -1           # scan of row 1 stops inside the third pass
    act_k = [5800]                   # ids in [5800, 6000) are skipped
    for kv_splits in (0, 3, 7):
        out, smax, ssum = sparse_flash_attention(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(si).to(dev),
                                                 scale_value=0.06, actual_seq_lengths_kv=act_k,
                                                 query_rope=qr.to(dev), key_rope=kr.to(dev), sparse_mode=mode,
                                                 return_softmax_lse=True, kv_splits=kv_splits)
        o = SFA.sparse_flash_attention(_np(q), _np(k), None, si, 0.06, None, None, act_k, _np(qr), _np(kr),
                                       1, "BSND", "BSND", mode, True, io_dtype="bf16")
        compare(out, smax, ssum, *o, what=f"long scan mode {mode} kv_splits={kv_splits}")


def test_split_rows_more_than_256_batches(dev):
    """KV-split decode rows over 300 batches (past the per-thread batch prefetch, so the
    batch is found by count and its lengths loaded directly), with skipped batches
    (act_q = 0) and short kv lengths; forced 2 splits."""
    B, N1, D, count, S2 = 300, 8, 128, 64, 96
    q, k, v, qr, kr = _inputs(B, 1, S2, N1, D, "bf16", seed=41)
    rng = np.random.RandomState(4)
    act_k = rng.randint(1, S2 + 1, size=B).tolist()
    act_q = [0 if b % 37 == 5 else 1 for b in range(B)]
    si = np.full((B, 1, 1, count), -1, dtype=np.int32)
    for b in range(B):
        n = min(count, act_k[b])
        si[b, 0, 0, :n] = np.sort(rng.permutation(act_k[b])[:n])
    out, smax, ssum = sparse_flash_attention(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(si).to(dev),
                                             scale_value=0.08, actual_seq_lengths_query=act_q,
                                             actual_seq_lengths_kv=act_k, query_rope=qr.to(dev),
                                             key_rope=kr.to(dev), sparse_mode=3, return_softmax_lse=True,
                                             kv_splits=2)
    o = SFA.sparse_flash_attention(_np(q), _np(k), None, si, 0.08, None, act_q, act_k, _np(qr), _np(kr), 1,
                                   "BSND", "BSND", 3, True, io_dtype="bf16")
    compare(out, smax, ssum, *o, what="300 batches, 2 splits")


@pytest.mark.parametrize("fill", [0x7F, 0xFF, "random"])
def test_workspace_contents_past_zero_prefix_are_ignored(dev, fill):
    """Only the workspace's zero prefix is cleared; the rest may hold anything. Decode
    rows whose KV splits list their own tokens (short splits: every tile is in the id
    ring's first four slots) must read only token-list positions written in the same
    call. Filled with far-out-of-range ids (0x7F7F7F7F), -1 and random bytes, then run
    twice on the same workspace."""
    from dsa_triton_ascend_amd.sparse_flash_attention import AttentionPlan
    from dsa_triton_ascend_amd import _lib
    B, S1, S2, N1, D, count = 1, 4, 2048, 8, 128, 2048
    q, k, v, qr, kr = _inputs(B, S1, S2, N1, D, "fp16")
    si = _ref_indices(B, S1, S2, count, 1, 3)
    o = SFA.sparse_flash_attention(_np(q), _np(k), None, si, 0.07, None, None, None, _np(qr), _np(kr), 1,
                                   "BSND", "BSND", 3, True, io_dtype="fp16")
    for kv_splits in (0, 16):
        plan = AttentionPlan(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(si).to(dev), scale_value=0.07,
                             query_rope=qr.to(dev), key_rope=kr.to(dev), sparse_mode=3,
                             return_softmax_lse=True, kv_splits=kv_splits)
        zb = _lib.load().dsa_sfa_workspace_zero_bytes()
        tail = plan.ws[zb:]
        if fill == "random":
            g = torch.Generator(device="cpu").manual_seed(11)
            tail.copy_(torch.randint(0, 256, (tail.numel(),), dtype=torch.uint8, generator=g))
        else:
            tail.fill_(fill)
        for rep in range(2):
            out, smax, ssum = plan.run()
            torch.cuda.synchronize()
            compare(out, smax, ssum, *o, what=f"workspace fill {fill} kv_splits={kv_splits} call {rep}")
