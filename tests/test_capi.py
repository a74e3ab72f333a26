"""C-ABI boundary checks that need no GPU: the library loads, exports every
symbol include/dsa_mi355x.h declares, and rejects invalid arguments with a
non-zero status and a message before touching the device; the Python entry
points raise the reference's ValueErrors before any device work."""
import ctypes
import re
from pathlib import Path

import pytest
import torch

from dsa_triton_ascend_amd import _lib
from dsa_triton_ascend_amd import lightning_indexer, sparse_flash_attention

HEADER = Path(__file__).resolve().parents[1] / "include" / "dsa_mi355x.h"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dsa_\w+)\s*\(", text)))


def test_header_symbols_exported():
    lib = _lib.load()
    syms = declared_symbols()
    assert {"dsa_li_score", "dsa_li_topk", "dsa_sfa_fwd", "dsa_sfa_workspace_bytes",
            "dsa_last_error", "dsa_abi_version"} <= set(syms)
    for s in syms:
        assert hasattr(lib, s), f"{s} declared in the header but not exported"
        assert s in _lib.SIGNATURES, f"{s} has no ctypes signature"
    assert lib.dsa_abi_version() == 1


def test_invalid_arguments_return_status_without_gpu():
    lib = _lib.load()
    st = lib.dsa_li_score(None, None, None, 1, 2, None, None, None, None, 1, 1, 8, 1, 128, 16,
                          1, 16, 3, None, 16, None)
    assert st == _lib.DSA_ERR_INVALID
    assert b"null pointer" in lib.dsa_last_error()
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    st = lib.dsa_li_score(p, p, p, 1, 2, p, p, p, p, 1, 1, 8, 3, 128, 16, 1, 16, 3, p, 16, None)
    assert st == _lib.DSA_ERR_INVALID and b"divisible" in lib.dsa_last_error()
    st = lib.dsa_li_score(p, p, p, 1, 2, p, p, p, p, 1, 1, 8, 1, 100, 16, 1, 16, 3, p, 16, None)
    assert st == _lib.DSA_ERR_UNSUPPORTED
    st = lib.dsa_li_topk(p, 70000, 1, p, p, p, 1, 1, 1, 70000, 3, 16385, p, None, None)
    assert st == _lib.DSA_ERR_UNSUPPORTED and b"16384" in lib.dsa_last_error()
    # above the LDS sort's cap: the workspace entry point sizes and checks its scratch
    assert lib.dsa_li_topk_workspace_bytes(4, 2, 70000, 16384) == 0
    assert lib.dsa_li_topk_workspace_bytes(4, 2, 70000, 16385) == 4 * 2 * 2 * 70000 * 8
    st = lib.dsa_li_topk_ws(p, 70000, 1, p, p, p, 1, 4, 2, 70000, 3, 16385, p, None, None, 0, None)
    assert st == _lib.DSA_ERR_INVALID and b"workspace" in lib.dsa_last_error()
    st = lib.dsa_li_topk_ws(p, 70000, 1, p, p, p, 1, 4, 2, 70000, 3, 16385, p, None, p,
                            4 * 2 * 2 * 70000 * 8 - 1, None)
    assert st == _lib.DSA_ERR_INVALID and b"workspace" in lib.dsa_last_error()
    base = [p, p, p, p, 1, p, 64, 1, None, 0, 0, p, p, p, p, 1, 1, 128, 512, 64, 16, 16, 3, 0.1,
            p, None, None, p, 1 << 30, 0, None]
    # `base` itself is valid and is never called: each case below breaks one field
    bad = list(base)
    bad[18] = 100
    assert lib.dsa_sfa_fwd(*bad) == _lib.DSA_ERR_INVALID and b"D must be one of" in lib.dsa_last_error()
    bad = list(base)
    bad[7] = 3
    assert lib.dsa_sfa_fwd(*bad) == _lib.DSA_ERR_INVALID and b"power of 2" in lib.dsa_last_error()
    bad = list(base)
    bad[17] = 96
    assert lib.dsa_sfa_fwd(*bad) == _lib.DSA_ERR_INVALID and b"N1 must be one of" in lib.dsa_last_error()
    bad = list(base)
    bad[22] = 1
    assert lib.dsa_sfa_fwd(*bad) == _lib.DSA_ERR_INVALID and b"sparse_mode" in lib.dsa_last_error()
    bad = list(base)
    bad[27], bad[28] = None, 0
    assert lib.dsa_sfa_fwd(*bad) == _lib.DSA_ERR_INVALID and b"workspace" in lib.dsa_last_error()
    bad = list(base)
    bad[29] = 17
    assert lib.dsa_sfa_fwd(*bad) == _lib.DSA_ERR_UNSUPPORTED and b"kv_splits" in lib.dsa_last_error()
    assert lib.dsa_sfa_workspace_bytes(4096, 128, 512, 2048, 1, 0) >= 4096 * 2048 * 4
    zb = lib.dsa_sfa_workspace_zero_bytes()
    assert zb >= (512 + 64) * 2 and zb % 256 == 0 and zb < lib.dsa_sfa_workspace_bytes(1, 1, 128, 1, 1, 1)


def test_python_validation_matches_reference():
    q = torch.zeros(1, 4, 8, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="block_table"):
        lightning_indexer(q, q[:, :, :1], torch.zeros(1, 4, 8), block_table=torch.zeros(1, 1))
    with pytest.raises(ValueError, match="requires block_table"):
        lightning_indexer(q, q[:, :, :1], torch.zeros(1, 4, 8), layout_key="PA_BSND")
    k = torch.zeros(1, 16, 1, 512, dtype=torch.bfloat16)
    qs = torch.zeros(1, 4, 8, 512, dtype=torch.bfloat16)
    qr = torch.zeros(1, 4, 8, 64, dtype=torch.bfloat16)
    kr = torch.zeros(1, 16, 1, 64, dtype=torch.bfloat16)
    si = torch.zeros(1, 4, 1, 8, dtype=torch.int32)
    cases = [(dict(attention_mode=1), "attention_mode"), (dict(sparse_mode=1), "sparse_mode"),
             (dict(pre_tokens=5), "pre_tokens"), (dict(sparse_block_size=3), "power of 2"),
             (dict(query_rope=None), "query_rope")]
    for kw, msg in cases:
        args = dict(query_rope=qr, key_rope=kr)
        args.update(kw)
        with pytest.raises(ValueError, match=msg):
            sparse_flash_attention(qs, k, k, si, **args)
    with pytest.raises(ValueError, match="block_table"):
        sparse_flash_attention(qs, k, k, si, query_rope=qr, key_rope=kr, layout_kv="PA_BSND")
    # CPU tensors are refused (no silent CPU path)
    with pytest.raises(ValueError, match="GPU"):
        sparse_flash_attention(qs, k, k, si, query_rope=qr, key_rope=kr)
    with pytest.raises(ValueError, match="GPU"):
        lightning_indexer(q, q[:, :, :1], torch.zeros(1, 4, 8))


def test_grad_validation_matches_reference():
    """The reference's guard cases (test_sfa_grad_triton.py:325-357) raise ValueError before
    any device work; CPU tensors are refused; the C ABI rejects bad shapes."""
    from dsa_triton_ascend_amd import sparse_flash_attention_grad
    q = torch.zeros(1, 4, 8, 512, dtype=torch.float16)
    k = torch.zeros(1, 128, 1, 512, dtype=torch.float16)
    qr = torch.zeros(1, 4, 8, 64, dtype=torch.float16)
    kr = torch.zeros(1, 128, 1, 64, dtype=torch.float16)
    si = torch.zeros(1, 4, 1, 64, dtype=torch.int32)
    sm = torch.zeros(1, 1, 4, 8)
    cases = [(dict(pre_tokens=0), "pre_tokens"), (dict(next_tokens=0), "next_tokens"),
             (dict(sparse_mode=1), "sparse_mode"), (dict(deterministic=True), "deterministic"),
             (dict(sparse_block_size=3), "power of 2"), (dict(query_rope=None), "query_rope")]
    for kw, msg in cases:
        args = dict(scale_value=0.04, query_rope=qr, key_rope=kr, sparse_mode=3)
        args.update(kw)
        with pytest.raises(ValueError, match=msg):
            sparse_flash_attention_grad(q, k, k, si, q, q, sm, sm, **args)
    with pytest.raises(ValueError, match="GPU"):
        sparse_flash_attention_grad(q, k, k, si, q, q, sm, sm, query_rope=qr, key_rope=kr)
    lib = _lib.load()
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    hrs = (ctypes.c_int32 * 2)(0, 4)
    hak = (ctypes.c_int32 * 1)(128)
    hp = lambda x: ctypes.cast(x, ctypes.c_void_p)
    base = [p, p, p, p, 1, p, 64, 1, p, p, p, p, hp(hrs), hp(hak), 1, 4, 8, 512, 64, 128, 128, 3, 0.04,
            p, p, p, p, p, p, p, p, p, p, 1 << 30, None]
    bad = list(base)
    bad[17] = 64
    assert lib.dsa_sfa_bwd(*bad) == _lib.DSA_ERR_INVALID and b"D must be one of" in lib.dsa_last_error()
    bad = list(base)
    bad[16] = 12
    assert lib.dsa_sfa_bwd(*bad) == _lib.DSA_ERR_INVALID and b"N1 must be one of" in lib.dsa_last_error()
    bad = list(base)
    bad[33] = 16
    assert lib.dsa_sfa_bwd(*bad) == _lib.DSA_ERR_INVALID and b"workspace" in lib.dsa_last_error()
    bad = list(base)
    bad[23] = None
    assert lib.dsa_sfa_bwd(*bad) == _lib.DSA_ERR_INVALID and b"null pointer" in lib.dsa_last_error()
    bad = list(base)
    bad[12] = None
    assert lib.dsa_sfa_bwd(*bad) == _lib.DSA_ERR_INVALID and b"null pointer" in lib.dsa_last_error()
    need = lib.dsa_sfa_bwd_workspace_bytes(1, hp(hrs), hp(hak), 128, 4, 8, 512, 64, 1, 128)
    # accumulators (128 key rows x (512 + 64 + 512) fp32) + two dense 128 x 64 buffers
    assert need >= 128 * (512 + 64 + 512) * 4 + 2 * 128 * 64 * 2 and need < (1 << 30)


def test_kl_loss_validation_matches_reference():
    """The reference's host guards (sparse_lightning_indexer_grad_kl_loss_triton.py:510-514)
    raise ValueError before any device work; CPU tensors are refused."""
    from dsa_triton_ascend_amd import sparse_lightning_indexer_grad_kl_loss as kl
    q = torch.zeros(1, 2, 8, 128, dtype=torch.float16)
    k = torch.zeros(1, 16, 1, 128, dtype=torch.float16)
    qi = torch.zeros(1, 2, 8, 128, dtype=torch.float16)
    ki = torch.zeros(1, 16, 1, 128, dtype=torch.float16)
    w = torch.zeros(1, 2, 8, dtype=torch.float16)
    si = torch.zeros(1, 2, 1, 4, dtype=torch.int32)
    sm = torch.zeros(1, 1, 2, 8)
    with pytest.raises(ValueError, match="BSND"):
        kl(q, k, qi, ki, w, si, sm, sm, layout="TND")
    with pytest.raises(ValueError, match="sparse_mode"):
        kl(q, k, qi, ki, w, si, sm, sm, sparse_mode=0)
    with pytest.raises(ValueError, match="Nidx2"):
        kl(q, k, qi, ki, w, si.reshape(1, 2, 4, 1), sm, sm)
    with pytest.raises(ValueError, match="GPU"):
        kl(q, k, qi, ki, w, si, sm, sm)
    lib = _lib.load()
    assert lib.dsa_sli_grad_workspace_bytes(1, 4, 2048, 1024, 128) >= 4 * 1024 * 4 + 2048 * 128 * 4


@pytest.mark.parametrize("bad,match", [
    ("weights", "weights must be"), ("query_index_b", "query_index must be"),
    ("query_index_s1", "query_index must be"), ("key_index_s2", "key_index must be"),
    ("key_index_d", "key_index must be"), ("sparse_indices_s1", "sparse_indices must be"),
    ("sparse_indices_b", "sparse_indices must be"), ("softmax_max", "softmax_max must be"),
    ("softmax_sum", "softmax_sum must be"), ("query_rope", "query_rope must be"),
    ("key_rope", "key_rope must be"), ("key_b", "key must be"), ("act_q", "actual_seq_qlen"),
    ("act_k", "actual_seq_klen")])
def test_kl_loss_shape_mismatch_raises_before_device(bad, match):
    """Every tensor the KL-loss kernels index by B * S1 rows or S2 keys is checked against
    query [B, S1, N1, D] and key [B, S2, 1, D] on the host, before the device check (CPU
    tensors throughout: the mismatch must be what raises)."""
    from dsa_triton_ascend_amd import sparse_lightning_indexer_grad_kl_loss as kl
    B, S1, S2, N1, D, G, Di, K = 2, 3, 16, 8, 128, 8, 128, 4
    z = lambda *s: torch.zeros(*s, dtype=torch.float16)
    t = dict(q=z(B, S1, N1, D), k=z(B, S2, 1, D), qi=z(B, S1, G, Di), ki=z(B, S2, 1, Di), w=z(B, S1, G),
             si=torch.zeros(B, S1, 1, K, dtype=torch.int32), smax=torch.zeros(B, 1, S1, N1),
             ssum=torch.zeros(B, 1, S1, N1), qr=z(B, S1, N1, 64), kr=z(B, S2, 1, 64))
    kw = {}
    wrong = {"weights": ("w", z(B, S1, G + 1)), "query_index_b": ("qi", z(B + 1, S1, G, Di)),
             "query_index_s1": ("qi", z(B, S1 + 1, G, Di)), "key_index_s2": ("ki", z(B, S2 - 1, 1, Di)),
             "key_index_d": ("ki", z(B, S2, 1, Di * 2)), "sparse_indices_s1": ("si", t["si"][:, :2]),
             "sparse_indices_b": ("si", t["si"][:1]), "softmax_max": ("smax", torch.zeros(B, 1, S1, N1 // 2)),
             "softmax_sum": ("ssum", torch.zeros(B, 1, S1 + 1, N1)), "query_rope": ("qr", z(B, S1, N1 // 2, 64)),
             "key_rope": ("kr", z(B, S2 + 1, 1, 64)), "key_b": ("k", z(B + 1, S2, 1, D))}
    if bad in wrong:
        name, val = wrong[bad]
        t[name] = val
    elif bad == "act_q":
        kw["actual_seq_qlen"] = [3, 3, 3]
    else:
        kw["actual_seq_klen"] = [16, 16, 16]
    with pytest.raises(ValueError, match=match):
        kl(t["q"], t["k"], t["qi"], t["ki"], t["w"], t["si"], t["smax"], t["ssum"], query_rope=t["qr"],
           key_rope=t["kr"], **kw)


def test_batch_lengths_broadcast_and_count():
    """One actual length applies to every batch (the reference's zeros[B] + lengths
    broadcast); other counts are refused."""
    from dsa_triton_ascend_amd import _host as H
    assert H.batch_lengths(None, 3, 7, "x") == [7, 7, 7]
    assert H.batch_lengths([5], 3, 7, "x") == [5, 5, 5]
    assert H.batch_lengths(torch.tensor([1, 2, 3]), 3, 7, "x") == [1, 2, 3]
    with pytest.raises(ValueError, match="3 per-batch lengths"):
        H.batch_lengths([1, 2], 3, 7, "x")


def test_dense_loss_validation_matches_reference():
    """The reference's dense checks (dense_loss_backward_triton.py:605-706, :745-760)
    raise before any device work; CPU tensors are refused; out-of-range shapes return
    DSA_ERR_UNSUPPORTED from the C ABI without touching the GPU."""
    from dsa_triton_ascend_amd import dense_lightning_indexer_softmax_lse as lse, dense_loss_backward as dl
    B, S1, S2 = 1, 2, 16
    q = torch.zeros(B, S1, 4, 128, dtype=torch.float16)
    k = torch.zeros(B, S2, 2, 128, dtype=torch.float16)
    qi = torch.zeros(B, S1, 32, 128, dtype=torch.float16)
    ki = torch.zeros(B, S2, 1, 128, dtype=torch.float16)
    w = torch.zeros(B, S1, 32, dtype=torch.float16)
    sm = torch.zeros(B, 2, S1, 2)
    with pytest.raises(ValueError, match="BSND"):
        lse(qi, ki, w, layout="TND")
    with pytest.raises(ValueError, match="Nidx1"):
        lse(qi[:, :, :8], ki, w[:, :, :8])
    with pytest.raises(ValueError, match="GPU"):
        lse(qi, ki, w)
    with pytest.raises(ValueError, match=r"\[B, N2, S1, G\]"):
        dl(q, k, qi, ki, w, sm[:, :1], sm[:, :1])
    with pytest.raises(ValueError, match="divisible"):
        dl(q, k[:, :, :1].expand(B, S2, 3, 128), qi, ki, w, sm, sm)
    with pytest.raises(ValueError, match="both provided"):
        dl(q, k, qi, ki, w, sm, sm, softmax_max_index=torch.zeros(B, 1, S1))
    with pytest.raises(ValueError, match="Drope"):
        dl(q, k, qi, ki, w, sm, sm, query_rope=torch.zeros(B, S1, 4, 32, dtype=torch.float16),
           key_rope=torch.zeros(B, S2, 2, 32, dtype=torch.float16))
    with pytest.raises(ValueError, match="GPU"):
        dl(q, k, qi, ki, w, sm, sm)
    lib = _lib.load()
    assert lib.dsa_dense_li_grad_workspace_bytes(1, 4, 2048, 128) >= 4 * 2048 * 4 + 2048 * 128 * 4
    one = ctypes.c_void_p(1)
    assert lib.dsa_dense_li_softmax_lse(one, one, one, 1, 1, one, one, 1, 4, 8192, 32, 64, one, one,
                                        None) == _lib.DSA_ERR_UNSUPPORTED   # D_idx = 64
    # rows of more than 4096 keys keep the index scores in the workspace: it grows by rows x S2 fp32
    assert (lib.dsa_dense_li_grad_workspace_bytes(1, 4, 8192, 128)
            >= lib.dsa_dense_li_grad_workspace_bytes(1, 4, 4096, 128) + 4 * 8192 * 4)
    assert lib.dsa_dense_li_grad_kl_loss(one, one, None, None, one, one, one, 1, 1, one, one, None, None, one,
                                         one, 1, 4, 64, 6, 4, 128, 0, 32, 128, 1.0, one, one, one, one, one,
                                         1 << 30, None) == _lib.DSA_ERR_INVALID   # N1 % N2
    assert b"divisible" in lib.dsa_last_error()


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(RuntimeError, match="missing"):
        _lib.load(tmp_path / "nope.so")


def test_noalloc_refuses_problems_beyond_the_scratch():
    """dsa_sfa_fwd_noalloc validates like dsa_sfa_fwd and refuses a problem whose workspace
    exceeds its static scratch, before any device work (no GPU needed)."""
    lib = _lib.load()
    one = ctypes.c_void_p(1)
    limit = 40 << 20   # DSA_SFA_NOALLOC_SCRATCH_BYTES
    # C5-sized prefill: 18216 rows x 2048 tokens of token lists alone exceed the scratch
    assert lib.dsa_sfa_workspace_bytes(18216, 128, 512, 2048, 1, 0) > limit
    args = [one, one, one, one, 1, one, 2048, 1, None, 0, 0, one, one, one, one, 4, 18216, 128, 512, 64, 8192,
            18216, 3, 0.04, one, one, one, 0, None]
    assert lib.dsa_sfa_fwd_noalloc(*args) == _lib.DSA_ERR_UNSUPPORTED
    assert b"static scratch" in lib.dsa_last_error()
    # C4 decode and C3 prefill fit
    assert lib.dsa_sfa_workspace_bytes(64, 128, 512, 2048, 1, 0) <= limit
    assert lib.dsa_sfa_workspace_bytes(4096, 128, 512, 2048, 1, 0) <= limit
    bad = list(args)
    bad[0] = None
    assert lib.dsa_sfa_fwd_noalloc(*bad) == _lib.DSA_ERR_INVALID and b"null pointer" in lib.dsa_last_error()
    bad = list(args)
    bad[18] = 64
    assert lib.dsa_sfa_fwd_noalloc(*bad) == _lib.DSA_ERR_INVALID and b"D must be" in lib.dsa_last_error()


def test_library_has_no_load_time_hipblaslt_dependency():
    """hipBLASLt (the SFA backward's library GEMMs) is loaded with dlopen on the first
    backward call: the indexer / forward library must load without it."""
    import subprocess
    out = subprocess.run(["readelf", "-d", str(_lib.LIB_PATH)], capture_output=True, text=True, check=True).stdout
    needed = re.findall(r"\(NEEDED\)\s+Shared library: \[([^\]]+)\]", out)
    assert needed, out
    assert not any("blas" in n for n in needed), needed


def test_grad_rejects_decreasing_host_row_start():
    """The host copies of the row offsets size and place the library GEMMs: an entry out
    of order is refused before any device work."""
    lib = _lib.load()
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    rs = (ctypes.c_int32 * 4)(0, 5, 3, 8)
    ak = (ctypes.c_int32 * 3)(64, 64, 64)
    st = lib.dsa_sfa_bwd(p, p, p, p, 1, p, 16, 1, p, p, p, p, ctypes.cast(rs, ctypes.c_void_p),
                         ctypes.cast(ak, ctypes.c_void_p), 3, 8, 8, 128, 64, 64, 192, 3, 0.1, p, p, p, p,
                         p, p, p, p, p, p, 1 << 30, None)
    assert st == _lib.DSA_ERR_INVALID and b"non-decreasing" in lib.dsa_last_error()
