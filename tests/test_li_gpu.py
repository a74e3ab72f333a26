"""GPU parity: lightning_indexer (HIP) vs the oracle (oracle/lightning_indexer_ref.py).

Shape matrix follows the reference's test_golden (test_li_triton.py:143-237):
GQA (N2 in {2,4}), odd N1=7, D in {64,96,128,256,512}, S1 != S2, B in {1,2},
fp16 and bf16. Rows of the larger cases are stride-sampled for the oracle;
size-independent invariants are checked on every row. Parity rule: see
tests/parity.py (bit-exact ordered indices and values, except bf16/fp16
rounding flips of scores within accumulation noise of a rounding midpoint).
"""
import numpy as np
import pytest
import torch

from dsa_triton_ascend_amd import LightningIndexer, lightning_indexer
from dsa_triton_ascend_amd import workloads as W
from oracle import lightning_indexer_ref as LI
from tests.parity import check_li, check_topk_properties

pytestmark = pytest.mark.gpu

DT = {"bf16": torch.bfloat16, "fp16": torch.float16}


def _inputs(B, S1, S2, N1, N2, D, dtype, seed=42, w_dtype=None, w_scale=1.0):
    """Reference test generator semantics (test_li_triton.py:30-36): randn -> 16-bit."""
    rng = np.random.RandomState(seed)
    t = DT[dtype]
    q = torch.from_numpy(rng.randn(B, S1, N1, D).astype(np.float32)).to(t)
    k = torch.from_numpy(rng.randn(B, S2, N2, D).astype(np.float32)).to(t)
    w = torch.from_numpy((rng.randn(B, S1, N1) * w_scale).astype(np.float32)).to(w_dtype or t)
    return q, k, w


def _np(t):
    return t.float().cpu().numpy()


def _rows(B, S1, max_rows):
    if B * S1 <= max_rows:
        return None
    stride = max(1, (B * S1) // max_rows)
    rows = [(b, s) for b in range(B) for s in range(S1) if (b * S1 + s) % stride == 0]
    rows += [(B - 1, S1 - 1), (0, 0)]
    return sorted(set(rows))


def _visible(S1, S2, aq, ak, mode):
    s1 = np.arange(S1)
    if mode == 3:
        L = np.minimum(np.minimum(np.maximum(ak - aq + s1 + 1, 0), S2), ak)
    else:
        L = np.full(S1, min(ak, S2))
    return np.where(s1 < aq, np.maximum(L, 0), 0)


def run_case(dev, B, S1, S2, N1, N2, D, K, mode=3, dtype="bf16", act_q=None, act_k=None,
             max_rows=96, w_dtype=None, w_scale=1.0):
    q, k, w = _inputs(B, S1, S2, N1, N2, D, dtype, w_dtype=w_dtype, w_scale=w_scale)
    idx, val = lightning_indexer(q.to(dev), k.to(dev), w.to(dev), actual_seq_lengths_query=act_q,
                                 actual_seq_lengths_key=act_k, sparse_count=K, sparse_mode=mode,
                                 return_value=True)
    torch.cuda.synchronize()
    assert idx.shape == (B, S1, N2, K) and idx.dtype == torch.int32
    assert val.shape == (B, S1, N2, K) and val.dtype == q.dtype
    gi, gv = idx.cpu().numpy(), val.float().cpu().numpy()
    aq = np.full(B, S1) if act_q is None else np.asarray(act_q)
    ak = np.full(B, S2) if act_k is None else np.asarray(act_k)
    Ls = np.concatenate([np.repeat(_visible(S1, S2, aq[b], ak[b], mode), N2) for b in range(B)])
    check_topk_properties(gi.reshape(-1, K), gv.reshape(-1, K), Ls, K)
    stats = check_li(gi, gv, _np(q), _np(k), _np(w), aq, ak, K, mode, dtype,
                     rows=_rows(B, S1, max_rows))
    print(f"[li parity] B={B} S1={S1} S2={S2} N1={N1} N2={N2} D={D} K={K} mode={mode} {dtype}: {stats}")
    # every flip is justified element by element; a kernel biased within E would
    # still show up as a high flip rate
    assert stats.flips <= max(4, 0.02 * stats.elements), stats
    return stats


GOLDEN_SHAPES = [
    (1, 128, 8, 1, 128, 32), (4, 256, 7, 1, 96, 32), (8, 128, 16, 2, 64, 64),
    (3, 256, 12, 4, 256, 32), (128, 128, 64, 1, 128, 64), (256, 512, 64, 1, 128, 128),
    (512, 256, 64, 1, 128, 128), (1024, 1024, 64, 1, 128, 512), (1024, 1024, 32, 1, 128, 512),
    (1024, 1024, 128, 1, 128, 512), (1024, 1024, 32, 1, 256, 512), (1024, 1024, 32, 1, 512, 512),
    (1024, 1024, 64, 1, 256, 512), (1024, 1024, 64, 1, 512, 512), (1024, 1024, 128, 1, 256, 512),
    (1024, 1024, 128, 1, 512, 512),
]


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("B", [1, 2])
@pytest.mark.parametrize("S1,S2,N1,N2,D,K", GOLDEN_SHAPES)
def test_golden_matrix(dev, S1, S2, N1, N2, D, K, B, dtype):
    run_case(dev, B, S1, S2, N1, N2, D, K, 3, dtype, max_rows=48)


def test_c1_full(dev):
    """BASELINE config 1, every row checked."""
    c = W.C1
    run_case(dev, 1, c["S1"], c["S2"], c["N1"], c["N2"], c["D"], c["sparse_count"], 3, "bf16",
             max_rows=10 ** 9, w_dtype=torch.float32, w_scale=1 / np.sqrt(8))


@pytest.mark.parametrize("mode", [0, 3])
@pytest.mark.parametrize("aq,ak", [(5, 40), (40, 5), (37, 64), (64, 37), (0, 64), (64, 0)])
def test_actual_lengths(dev, mode, aq, ak):
    run_case(dev, 2, 64, 64, 16, 1, 128, 24, mode, "bf16", act_q=[aq, 64], act_k=[ak, 31],
             max_rows=10 ** 9)


def test_sparse_count_larger_than_s2(dev):
    run_case(dev, 1, 16, 40, 8, 1, 64, 64, 3, "bf16", max_rows=10 ** 9)


def test_return_value_false_and_module(dev):
    q, k, w = _inputs(1, 32, 32, 8, 1, 128, "bf16")
    mod = LightningIndexer(sparse_count=8, sparse_mode=3, return_value=False)
    idx, val = mod(q.to(dev), k.to(dev), w.to(dev))
    i2, _ = lightning_indexer(q.to(dev), k.to(dev), w.to(dev), sparse_count=8, return_value=True)
    assert torch.equal(idx, i2) and not val.any() and val.dtype == torch.bfloat16


@pytest.mark.parametrize("w_dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_weight_dtypes(dev, w_dtype):
    run_case(dev, 1, 48, 48, 16, 2, 64, 16, 3, "bf16", w_dtype=w_dtype, max_rows=10 ** 9)


@pytest.mark.parametrize("layout_key", ["TND", "BSND"])
def test_tnd(dev, layout_key):
    lens_q = [7, 33, 1, 64]
    lens_k = [7, 40, 5, 64] if layout_key == "TND" else [64, 64, 64, 64]
    N1, N2, D, K = 16, 1, 128, 16
    rng = np.random.RandomState(3)
    T1 = sum(lens_q)
    q = torch.from_numpy(rng.randn(T1, N1, D).astype(np.float32)).bfloat16()
    if layout_key == "TND":
        k = torch.from_numpy(rng.randn(sum(lens_k), N2, D).astype(np.float32)).bfloat16()
    else:
        k = torch.from_numpy(rng.randn(4, 64, N2, D).astype(np.float32)).bfloat16()
    w = torch.from_numpy(rng.randn(T1, N1).astype(np.float32))
    cu_q, cu_k = np.cumsum(lens_q).tolist(), np.cumsum(lens_k).tolist()
    idx, val = lightning_indexer(q.to(dev), k.to(dev), w.to(dev), cu_q, cu_k, layout_query="TND",
                                 layout_key=layout_key, sparse_count=K, sparse_mode=3,
                                 return_value=True)
    assert idx.shape == (T1, N2, K)
    o_idx, o_val = LI.lightning_indexer(_np(q), _np(k), _np(w), cu_q, cu_k, layout_query="TND",
                                        layout_key=layout_key, sparse_count=K, sparse_mode=3,
                                        return_value=True)
    gi, gv = idx.cpu().numpy(), val.float().cpu().numpy()
    # exact agreement expected at these sizes; fall back to the rounding-aware check per row
    if not (np.array_equal(gi, o_idx) and np.array_equal(gv, o_val)):
        from tests.parity import check_li_row, LiParityStats, row_error_bound
        act_q = np.diff([0] + cu_q)
        act_k = np.diff([0] + cu_k)
        stats = LiParityStats()
        qb = LI.tnd_to_bsnd(_np(q), act_q)
        wb = LI.tnd_to_bsnd(_np(w), act_q)
        kb = LI.tnd_to_bsnd(_np(k), act_k) if layout_key == "TND" else _np(k)
        r = 0
        for b in range(4):
            for s in range(act_q[b]):
                s32 = LI.li_row_scores(qb, kb, wb, b, s, 0, act_q, act_k, 3)
                s64 = LI.li_row_scores_f64(qb, kb, wb, b, s, 0, act_q, act_k, 3)
                err = row_error_bound(qb, kb, wb, b, s, 0)
                check_li_row(gi[r, 0], gv[r, 0], s32, s64, int(act_k[b]), K, "bf16", stats, err=err)
                r += 1
        assert stats.flips <= max(4, 0.02 * stats.elements), stats


@pytest.mark.slow
def test_c2_full_size_sampled(dev):
    """BASELINE config 2 (1x8192, 64 heads, k=2048): invariants on all 8192 rows,
    oracle parity on a stride sample spanning the causal triangle."""
    c = W.C2
    inp = W.indexer_inputs(**{k: v for k, v in c.items()}, device=dev, seed=42)
    idx, val = lightning_indexer(inp.query, inp.key, inp.weights, sparse_count=c["sparse_count"],
                                 sparse_mode=3, return_value=True)
    torch.cuda.synchronize()
    K, S = c["sparse_count"], c["S1"]
    gi = idx.cpu().numpy()
    gv = val.float().cpu().numpy()
    check_topk_properties(gi.reshape(-1, K), gv.reshape(-1, K), np.arange(1, S + 1), K)
    rows = [(0, s) for s in list(range(0, S, 257)) + [2046, 2047, 2048, S - 1]]
    stats = check_li(gi, gv, _np(inp.query), _np(inp.key), _np(inp.weights), [S], [S], K, 3,
                     "bf16", rows=rows)
    print(f"[li parity C2] {stats}")
    assert stats.flips <= max(4, 0.01 * stats.elements), stats


@pytest.mark.slow
@pytest.mark.parametrize("S1,S2", [(4096, 4096), (4096, 8192), (16384, 16384)])
def test_reference_production_shapes(dev, S1, S2):
    """The reference's production shapes (test_li_triton.py:49-51): 4096 x 4096, S2 > S1
    (non-square causal, the reference's grid-overflow regression point) and 16K x 16K, 64
    heads, D=128, top-2048: top-k invariants on every row, oracle parity on stride-sampled
    rows spanning the causal triangle."""
    run_case(dev, 1, S1, S2, 64, 1, 128, 2048, 3, "bf16", max_rows=48)


@pytest.mark.parametrize("mode", [0, 3])
def test_rows_longer_than_register_cache(dev, mode):
    """S2 = 12,000 > 8,192: the top-k streams a row's keys from memory in two chunks (the
    histogram passes, the compaction and its cross-chunk offsets)."""
    run_case(dev, 1, 16, 12000, 8, 1, 64, 512, mode, "bf16", max_rows=10 ** 9)


@pytest.mark.parametrize("S2,K", [(131072, 2048), (131072, 16384), (70000, 9000)])
def test_long_context_rows(dev, S2, K):
    """DeepSeek-V3.2's 128K context: 16 query rows at the end of a 131,072-key causal window
    (each row sees 131,057 .. 131,072 keys; 32-bit indices, rows streamed in 16 chunks),
    top-k 2048 and 16384 (the largest sparse_count, 64 keys per thread in the sort), and a
    row length that is no multiple of the 8192-key chunk. Oracle on 6 of the rows, the
    top-k invariants on all."""
    B, S1, N1, N2, D = 1, 16, 64, 1, 128
    run_case(dev, B, S1, S2, N1, N2, D, K, 3, "bf16", act_q=[S1], act_k=[S2], max_rows=4, w_scale=1 / 8)


@pytest.mark.parametrize("S2,K,mode", [(20000, 18000, 3), (70000, 40000, 0), (17000, 17000, 3)])
def test_sparse_count_above_the_lds_sort(dev, S2, K, mode):
    """sparse_count > 16,384 (the reference's mint.topk path has no cap): every visible entry of
    a row is sorted in global scratch (dsa_li_topk_ws), 32-bit indices past 65,535 included,
    and rows shorter than k (the 17,000-key case) pad with -1. Oracle on sampled rows, the
    top-k invariants on all."""
    B, S1, N1, N2, D = 1, 8, 8, 1, 64
    run_case(dev, B, S1, S2, N1, N2, D, K, mode, "bf16", act_q=[S1], act_k=[S2], max_rows=4, w_scale=1 / 8)


def test_pa_bsnd_128k_context(dev):
    """Decode-time indexing over a 128K paged context with 32-token pages (4,097 block-table
    entries per batch), one query row per batch."""
    rng = np.random.RandomState(14)
    B, N1, D, K, dtype, page = 2, 64, 128, 2048, "bf16", 32
    lens = [131072, 100003]
    bt, cache, dense = _paged(rng, B, lens, page, 1, D, dtype, spare=1)
    q = torch.from_numpy(rng.randn(B, 1, N1, D).astype(np.float32)).to(DT[dtype])
    w = torch.from_numpy(rng.randn(B, 1, N1).astype(np.float32) / 8).to(DT[dtype])
    idx, val = lightning_indexer(q.to(dev), cache.to(dev), w.to(dev), actual_seq_lengths_key=lens,
                                 block_table=bt.to(dev), layout_key="PA_BSND", sparse_count=K, sparse_mode=3,
                                 return_value=True)
    torch.cuda.synchronize()
    gi, gv = idx.cpu().numpy(), val.float().cpu().numpy()
    S2 = dense.shape[1]
    Ls = np.array([min(l, S2) for l in lens])
    check_topk_properties(gi.reshape(-1, K), gv.reshape(-1, K), Ls, K)
    stats = check_li(gi, gv, _np(q), dense, _np(w), np.ones(B, int), np.asarray(lens), K, 3, dtype)
    print(f"[li parity] PA 128K: {stats}")
    assert stats.flips <= max(4, 0.02 * stats.elements), stats
    assert gi.max() >= 65536   # indices past 16 bits are produced


def test_heavy_ties_at_the_threshold(dev):
    """Keys repeat four distinct rows, so each score row holds only a few distinct values
    and the k-th largest sits inside a large run of ties (taken in index order)."""
    B, S1, S2, N1, N2, D, K = 1, 24, 700, 8, 1, 64, 100
    q, k, w = _inputs(B, S1, S2, N1, N2, D, "bf16", seed=3)
    k = k[:, :4].repeat(1, S2 // 4 + 1, 1, 1)[:, :S2].contiguous()
    idx, val = lightning_indexer(q.to(dev), k.to(dev), w.to(dev), sparse_count=K, sparse_mode=0,
                                 return_value=True)
    torch.cuda.synchronize()
    gi, gv = idx.cpu().numpy(), val.float().cpu().numpy()
    Ls = np.full(B * S1 * N2, S2)
    check_topk_properties(gi.reshape(-1, K), gv.reshape(-1, K), Ls, K)
    stats = check_li(gi, gv, _np(q), _np(k), _np(w), np.full(B, S1), np.full(B, S2), K, 0, "bf16")
    print(f"[li parity] heavy ties: {stats}")
    assert stats.flips <= max(4, 0.02 * stats.elements), stats


def _paged(rng, B, lens, page, N2, D, dtype, missing=None, spare=3):
    """Random paged key cache for per-batch kv lengths: a block table [B, max_blocks] over a
    shuffled pool (-1 past each batch's blocks and at `missing` = (b, i)), the cache
    [pool, page, N2, D] and the same keys de-paged by hand [B, max_blocks * page, N2, D]."""
    nb = [(l + page - 1) // page for l in lens]
    max_blocks = max(nb) + 1
    pool = sum(nb) + spare
    perm = rng.permutation(pool)
    bt = np.full((B, max_blocks), -1, np.int32)
    off = 0
    for b in range(B):
        bt[b, :nb[b]] = perm[off:off + nb[b]]
        off += nb[b]
    if missing is not None:
        bt[missing] = -1
    cache = torch.from_numpy(rng.randn(pool, page, N2, D).astype(np.float32)).to(DT[dtype])
    c = cache.float().numpy()
    dense = np.zeros((B, max_blocks * page, N2, D), np.float32)
    for b in range(B):
        for i in range(max_blocks):
            if bt[b, i] >= 0:
                dense[b, i * page:(i + 1) * page] = c[bt[b, i]]
    return torch.from_numpy(bt), cache, dense


@pytest.mark.parametrize("mode", [0, 3])
@pytest.mark.parametrize("page", [16, 48, 64])
def test_pa_bsnd_keys(dev, mode, page):
    """Keys from a paged cache (an extension: the reference rejects block_table). Parity
    with the golden on the keys de-paged by hand; a missing (-1) block inside a batch's
    range is a zero key row (score 0); non-power-of-two pages."""
    rng = np.random.RandomState(12)
    B, S1, N1, N2, D, K, dtype = 3, 4, 32, 1, 128, 64, "bf16"
    lens = [200, 77, 511]
    bt, cache, dense = _paged(rng, B, lens, page, N2, D, dtype, missing=(0, 1))
    q = torch.from_numpy(rng.randn(B, S1, N1, D).astype(np.float32)).to(DT[dtype])
    w = torch.from_numpy(rng.randn(B, S1, N1).astype(np.float32)).to(DT[dtype])
    idx, val = lightning_indexer(q.to(dev), cache.to(dev), w.to(dev), actual_seq_lengths_key=lens,
                                 block_table=bt.to(dev), layout_key="PA_BSND", sparse_count=K,
                                 sparse_mode=mode, return_value=True)
    torch.cuda.synchronize()
    gi, gv = idx.cpu().numpy(), val.float().cpu().numpy()
    S2 = dense.shape[1]
    aq, ak = np.full(B, S1), np.asarray(lens)
    Ls = np.concatenate([_visible(S1, S2, aq[b], ak[b], mode) for b in range(B)])
    check_topk_properties(gi.reshape(-1, K), gv.reshape(-1, K), Ls, K)
    stats = check_li(gi, gv, _np(q), dense, _np(w), aq, ak, K, mode, dtype)
    assert stats.flips <= max(4, 0.02 * stats.elements), stats
    # the oracle's own de-paging agrees with the hand-built one
    o_idx, _ = LI.lightning_indexer(_np(q), cache.float().numpy(), _np(w), None, lens, bt.numpy(), "BSND",
                                    "PA_BSND", K, mode, True, value_dtype=dtype)
    assert (o_idx == gi).mean() > 0.97


def test_pa_bsnd_decode_shape(dev):
    """Decode-time indexing: one query row per batch, 64 heads, kv lengths in the
    thousands over 128-token pages (the SFA decode cache layout), TND queries."""
    rng = np.random.RandomState(13)
    B, N1, D, K, dtype, page = 8, 64, 128, 2048, "bf16", 128
    lens = rng.randint(2500, 9000, size=B).tolist()
    bt, cache, dense = _paged(rng, B, lens, page, 1, D, dtype)
    q = torch.from_numpy(rng.randn(B, N1, D).astype(np.float32)).to(DT[dtype])
    w = torch.from_numpy(rng.randn(B, N1).astype(np.float32) / 8).to(DT[dtype])
    cq = list(range(1, B + 1))
    idx, val = lightning_indexer(q.to(dev), cache.to(dev), w.to(dev), actual_seq_lengths_query=cq,
                                 actual_seq_lengths_key=lens, block_table=bt.to(dev), layout_query="TND",
                                 layout_key="PA_BSND", sparse_count=K, sparse_mode=3, return_value=True)
    torch.cuda.synchronize()
    gi, gv = idx.cpu().numpy().reshape(B, 1, 1, K), val.float().cpu().numpy().reshape(B, 1, 1, K)
    S2 = dense.shape[1]
    Ls = np.array([min(l, S2) for l in lens])
    check_topk_properties(gi.reshape(-1, K), gv.reshape(-1, K), Ls, K)
    stats = check_li(gi, gv, _np(q).reshape(B, 1, N1, D), dense, _np(w).reshape(B, 1, N1), np.ones(B, int),
                     np.asarray(lens), K, 3, dtype)
    assert stats.flips <= max(4, 0.02 * stats.elements), stats


def _crafted_bits(family, rows, S2, rng):
    """16-bit bf16 patterns of a crafted score matrix [rows, S2] (uint16)."""
    f32 = dict(dtype=np.float32)
    if family == "equal":   # one value: no sort pass runs
        return np.full((rows, S2), 0x3F80, np.uint16)
    if family == "signed_zeros":   # +0 / -0 (equal keys) with a few real values
        b = np.where(rng.random((rows, S2), **f32) < 0.5, 0x0000, 0x8000).astype(np.uint16)
        x = ((rng.standard_normal((rows, S2), **f32) * 0.1).view(np.uint32) >> 16).astype(np.uint16)
        return np.where(rng.random((rows, S2), **f32) < 0.05, x, b)
    if family == "extremes":   # +inf, the largest finite values, subnormals, both signs
        pool = np.array([0x7F80, 0x7F7F, 0xFF7F, 0x0001, 0x8001, 0x3F80, 0xBF80, 0x0000], np.uint16)
        return pool[rng.integers(0, len(pool), (rows, S2))]
    if family == "two_values":   # adjacent keys: the threshold sits in a long run of ties
        return np.where(rng.random((rows, S2), **f32) < 0.5, 0x3F80, 0x3F81).astype(np.uint16)
    if family == "wide":   # both signs over forty binades: every digit pass runs
        x = rng.standard_normal((rows, S2), **f32) * np.exp2(rng.uniform(-20, 20, (rows, S2))).astype(np.float32)
        return (x.view(np.uint32) >> 16).astype(np.uint16)
    if family == "narrow":   # a few dozen keys either side of a 16-key digit boundary
        key = 0xBF80 + rng.integers(-24, 24, (rows, S2))   # ord16 keys of positive values
        return (key & 0x7FFF).astype(np.uint16)
    raise ValueError(family)


@pytest.mark.parametrize("S1,S2,K", [(8192, 8192, 2048), (64, 12000, 2048), (8, 70000, 2048),
                                     (16, 20000, 18000), (8, 70000, 40000)])
@pytest.mark.parametrize("family", ["equal", "signed_zeros", "extremes", "two_values", "wide", "narrow"])
def test_topk_crafted_score_rows(dev, S1, S2, K, family):
    """The top-k kernel alone on crafted score rows, against the golden's stable sort
    (oracle select_topk): ties, +0/-0, infinities and subnormals, rows of one value
    (no digit pass), both signs over many binades (every pass), and rows of every
    visible length around k, in the register-cached (S2 <= 8192), chunked and 32-bit
    index paths, and with k above the LDS sort's cap (sorted in global scratch). -inf is
    left out: the golden drops -inf entries (its mask value)."""
    from dsa_triton_ascend_amd.lightning_indexer import IndexerPlan
    rng = np.random.default_rng(11)
    q = torch.zeros(1, S1, 8, 128, dtype=torch.bfloat16, device=dev)
    k = torch.zeros(1, S2, 1, 128, dtype=torch.bfloat16, device=dev)
    w = torch.zeros(1, S1, 8, dtype=torch.float32, device=dev)
    plan = IndexerPlan(q, k, w, sparse_count=K, sparse_mode=3, return_value=True)
    bits = _crafted_bits(family, S1, S2, rng)
    sc = torch.from_numpy(bits.view(np.int16)).to(dev)
    plan.scores.zero_()
    plan.scores[:S1, :S2] = sc
    plan.topk()
    torch.cuda.synchronize()
    gi = plan.idx.reshape(S1, K).cpu().numpy()
    gv = plan.vals.reshape(S1, K).float().cpu().numpy()
    vals = (bits.astype(np.uint32) << 16).view(np.float32)
    rows = sorted({0, 1, 2, 63, 64, 255, 1023, 2046, 2047, 2048, 2049, 3000, 4095, 4096, 6143,
                   6144, 8190, 8191} | set(range(0, S1, 97)))
    rows = [r for r in rows if r < S1]
    for r in rows:
        L = S2 - S1 + r + 1
        s = np.full(S2, -np.inf, np.float32)
        s[:L] = vals[r, :L]
        ei, ev = LI.select_topk(s, S2, K)
        assert np.array_equal(gi[r], ei), (family, S2, r, L, np.flatnonzero(gi[r] != ei)[:8])
        assert np.array_equal(gv[r], ev), (family, S2, r, L)


@pytest.mark.parametrize("S1,S2,K", [(4096, 4096, 2048), (16, 20000, 2048), (8, 70000, 2048)])
def test_topk_order_of_nan_and_signed_zero_patterns(dev, S1, S2, K):
    """Bit patterns outside the golden's contract (NaNs), next to +-0 and +-inf: the top-k
    orders every 16-bit pattern as sign-magnitude (0x8000 + m / 0x8000 - m), so negative
    NaNs fall below -inf (0xFFFF lowest of all) and positive ones above +inf, +0 ties -0
    and a -0 comes back as +0. Expected order: a numpy stable sort on that key, rows with
    L <= k and L > k, in the register-cached, chunked and 32-bit index paths."""
    from dsa_triton_ascend_amd.lightning_indexer import IndexerPlan
    rng = np.random.default_rng(5)
    q = torch.zeros(1, S1, 8, 128, dtype=torch.bfloat16, device=dev)
    k = torch.zeros(1, S2, 1, 128, dtype=torch.bfloat16, device=dev)
    w = torch.zeros(1, S1, 8, dtype=torch.float32, device=dev)
    plan = IndexerPlan(q, k, w, sparse_count=K, sparse_mode=3, return_value=True)
    pool = np.array([0xFFFF, 0xFFC0, 0xFF81, 0x7FC0, 0x7F81, 0x7FFF, 0xFF80, 0x7F80, 0x0000, 0x8000],
                    np.uint16)
    normal = ((rng.standard_normal((S1, S2), dtype=np.float32)).view(np.uint32) >> 16).astype(np.uint16)
    bits = np.where(rng.random((S1, S2)) < 0.3, pool[rng.integers(0, len(pool), (S1, S2))], normal)
    plan.scores.zero_()
    plan.scores[:S1, :S2] = torch.from_numpy(bits.view(np.int16)).to(dev)
    plan.topk()
    torch.cuda.synchronize()
    gi = plan.idx.reshape(S1, K).cpu().numpy()
    gv = plan.vals.reshape(S1, K).view(torch.int16).cpu().numpy().view(np.uint16)
    m = bits.astype(np.int64) & 0x7FFF
    key = np.where(bits & 0x8000, 0x8000 - m, 0x8000 + m)
    rows = sorted({0, 1, 2047, 2048, 2049, 3000, S1 - 1} | set(range(0, S1, 257)))
    for r in (r for r in rows if r < S1):
        L = S2 - S1 + r + 1
        order = np.lexsort((np.arange(L), -key[r, :L]))[:min(L, K)]
        n = len(order)
        assert np.array_equal(gi[r, :n], order), (S2, r, L, np.flatnonzero(gi[r, :n] != order)[:8])
        assert np.all(gi[r, n:] == -1)
        ev = np.where(bits[r, order] == 0x8000, 0, bits[r, order])
        assert np.array_equal(gv[r, :n], ev), (S2, r, L)
        assert np.all(gv[r, n:] == 0)
