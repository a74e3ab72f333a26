"""dsa_sfa_fwd_noalloc: the sparse flash attention forward on the library's static
per-device scratch instead of a caller workspace (include/dsa_mi355x.h).

It runs the kernels of dsa_sfa_fwd, so its outputs must equal that entry point's bit for
bit on the same inputs; every call shares the device's scratch, so two calls in a row
(the second smaller, on the contents the first left behind) must both match. Output
buffers start as NaN so an unwritten element shows. Also checked against the oracle.
"""
import numpy as np
import pytest
import torch

from dsa_triton_ascend_amd import _host as H
from dsa_triton_ascend_amd import _lib
from dsa_triton_ascend_amd import workloads as W
from dsa_triton_ascend_amd.sparse_flash_attention import AttentionPlan
from oracle import sparse_flash_attention_ref as SFA

pytestmark = pytest.mark.gpu


def _noalloc(plan):
    """One dsa_sfa_fwd_noalloc call with the validated arguments of an AttentionPlan,
    into fresh NaN-filled outputs."""
    out = torch.full_like(plan.out, float("nan"))
    smax = torch.full_like(plan.sm_max, float("nan"))
    ssum = torch.full_like(plan.sm_sum, float("nan"))
    lib = _lib.load()
    st = lib.dsa_sfa_fwd_noalloc(
        plan.q.data_ptr(), plan.qr.data_ptr(), plan.kk.data_ptr(), plan.kr.data_ptr(), plan.io,
        plan.si.data_ptr(), plan.count, plan.sbs, H.ptr(plan.d_bt), plan.max_blocks, plan.page_bs,
        plan.d_row_start.data_ptr(), plan.d_key_start.data_ptr(), plan.d_aq.data_ptr(), plan.d_ak.data_ptr(),
        plan.B, plan.total_rows, plan.N1, plan.D, plan.Dr, plan.S2, plan.key_rows, plan.sparse_mode, plan.scale,
        out.data_ptr(), smax.data_ptr(), ssum.data_ptr(), plan.kv_splits, H.stream_ptr(plan.dev))
    _lib.check(st, "dsa_sfa_fwd_noalloc")
    return out, smax, ssum


def _decode(dev, B, N1, lens, block, count, seed):
    inp = W.sfa_decode_inputs(B=B, N1=N1, len_lo=lens[0], len_hi=lens[1], block_size=block,
                              sparse_count=count, device="cpu", seed=seed)
    bt = inp.block_table.clone()
    bt[1, 1] = -1   # a missing page: its tokens read the scratch's zero row
    plan = AttentionPlan(inp.query.to(dev), inp.key.to(dev), inp.key.to(dev), inp.sparse_indices.to(dev),
                         scale_value=inp.scale_value, block_table=bt.to(dev),
                         actual_seq_lengths_kv=inp.actual_seq_lengths_kv, query_rope=inp.query_rope.to(dev),
                         key_rope=inp.key_rope.to(dev), layout_kv="PA_BSND", sparse_mode=3,
                         return_softmax_lse=True, block_size=block)
    return inp, bt, plan


def _oracle(inp, bt, block):
    f = lambda t: t.float().cpu().numpy()
    return SFA.sparse_flash_attention(f(inp.query), f(inp.key), None, inp.sparse_indices.numpy(), inp.scale_value,
                                      bt.numpy(), None, inp.actual_seq_lengths_kv, f(inp.query_rope),
                                      f(inp.key_rope), 1, "BSND", "PA_BSND", 3, True, block_size=block,
                                      io_dtype="bf16")


def _check(got, want_plan, oracle, what):
    for name, g, w in zip(("out", "softmax_max", "softmax_sum"), got, want_plan):
        assert torch.equal(g, w), f"{what}: {name} differs from dsa_sfa_fwd"
    go = got[0].float().cpu().numpy()
    assert np.all(np.isfinite(go))
    np.testing.assert_allclose(go, oracle[0], rtol=1e-2, atol=1e-2, err_msg=f"{what}: out vs oracle")
    np.testing.assert_allclose(got[2].cpu().numpy(), oracle[2], rtol=1e-4, atol=1e-5,
                               err_msg=f"{what}: softmax_sum vs oracle")


def test_noalloc_matches_workspace_entry_two_calls(dev):
    """A paged decode call (32 rows over 2048 tokens, KV splits listing their own tokens,
    split partials in the scratch), then a smaller one (4 rows, 256 tokens)."""
    big = _decode(dev, 32, 128, (2048, 8192), 64, 2048, seed=5)
    small = _decode(dev, 4, 64, (300, 900), 64, 256, seed=6)
    for (inp, bt, plan), what, block in ((big, "32 rows x 2048", 64), (small, "4 rows x 256", 64)):
        got = _noalloc(plan)
        want = plan.run()
        torch.cuda.synchronize()
        _check(got, want, _oracle(inp, bt, block), what)
    # the first problem again, on the contents the second left in the scratch
    got = _noalloc(big[2])
    torch.cuda.synchronize()
    _check(got, big[2].run(), _oracle(big[0], big[1], 64), "32 rows x 2048 again")


def test_noalloc_prefill_token_lists(dev):
    """Unsplit prefill rows (the token-list kernel writes the scratch's token lists),
    then a smaller problem."""
    for S, N1, count in ((256, 32, 128), (64, 16, 32)):
        inp = W.sfa_prefill_inputs(B=1, S1=S, S2=S, N1=N1, D=512, sparse_count=count, device="cpu", seed=S)
        plan = AttentionPlan(inp.query.to(dev), inp.key.to(dev), inp.key.to(dev), inp.sparse_indices.to(dev),
                             **{k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in inp.kwargs().items()})
        got = _noalloc(plan)
        want = plan.run()
        torch.cuda.synchronize()
        f = lambda t: t.float().cpu().numpy()
        o = SFA.sparse_flash_attention(f(inp.query), f(inp.key), None, inp.sparse_indices.numpy(), inp.scale_value,
                                       query_rope=f(inp.query_rope), key_rope=f(inp.key_rope), sparse_mode=3,
                                       return_softmax_lse=True, io_dtype="bf16")
        _check(got, want, o, f"prefill S={S}")
