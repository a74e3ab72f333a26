"""Seeded synthetic inputs for the five benchmark / parity configurations.

C1  lightning_indexer BSND 1x256, N1=8, D=128, k=64, causal (the reference's CPU shape)
C2  lightning_indexer BSND 1x8192, N1=64, D=128, k=2048, causal (DeepSeek-V3.2 prefill)
C3  sparse_flash_attention BSND 1x4096, N1=128, D=512+64, top-k 2048, causal, LSE on
C4  sparse_flash_attention PA_BSND decode, block 128, B=64, kv lengths U[4096, 32768]
C5  TND pipeline: lengths {1024, 3000, 6000, 8192}, indexer (64 heads) feeding SFA (128 heads)
GRAD_PERF  sparse_flash_attention_grad BSND 1x512 over 4096 keys, N1=64, D=512+64, top-k 2048

All shapes are parameters so tests can run scaled-down versions. Tensors are
drawn with a ``torch.Generator`` (on the CPU for tests, on the device for the
bench) from N(0,1) in float32 and rounded once to the io dtype (RNE).
Sparse-index construction follows the reference generator
(test_sfa_triton.py:64-85): front-valid sorted distinct positions inside each
row's causal window, -1 padded at the back.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch


def _gen(device, seed):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def _randn(shape, g, device, dtype, scale=1.0):
    x = torch.randn(shape, generator=g, device=device, dtype=torch.float32)
    if scale != 1.0:
        x = x * scale
    return x.to(dtype)


def sorted_random_subsets(limits, count, g, device, max_pos=None):
    """For each row r pick ``min(limits[r], count)`` distinct positions in
    ``[0, limits[r])`` uniformly at random, sorted ascending, padded with -1.

    limits: int64 tensor [R]. Returns int32 [R, count]."""
    R = limits.shape[0]
    if max_pos is None:
        max_pos = int(limits.max().item()) if R else 0
    max_pos = max(max_pos, count)
    out = torch.empty((R, count), dtype=torch.int32, device=device)
    step = max(1, (1 << 26) // max_pos)          # bound the [rows, max_pos] scratch to 256 MiB
    pos = torch.arange(max_pos, device=device)
    for r0 in range(0, R, step):
        lim = limits[r0:r0 + step].to(device)
        keys = torch.rand((lim.shape[0], max_pos), generator=g, device=device)
        keys = torch.where(pos[None, :] < lim[:, None], keys, torch.full_like(keys, 2.0))
        sel = torch.topk(keys, count, dim=1, largest=False).indices
        sel = torch.where(sel < lim[:, None], sel, torch.full_like(sel, 1 << 30))
        sel = torch.sort(sel, dim=1).values
        out[r0:r0 + step] = torch.where(sel >= (1 << 30), torch.full_like(sel, -1), sel).to(torch.int32)
    return out


@dataclass
class IndexerInputs:
    query: torch.Tensor
    key: torch.Tensor
    weights: torch.Tensor
    sparse_count: int
    sparse_mode: int = 3
    layout: str = "BSND"
    actual_seq_lengths_query: object = None
    actual_seq_lengths_key: object = None


def indexer_inputs(B=1, S1=256, S2=256, N1=8, N2=1, D=128, sparse_count=64, sparse_mode=3,
                   w_scale=None, dtype=torch.bfloat16, w_dtype=torch.float32, device="cpu", seed=42):
    """BSND indexer inputs (C1 defaults; C2 = S1=S2=8192, N1=64, k=2048, w_scale=1/8)."""
    g = _gen(device, seed)
    if w_scale is None:
        w_scale = 1.0 / math.sqrt(N1)
    q = _randn((B, S1, N1, D), g, device, dtype)
    k = _randn((B, S2, N2, D), g, device, dtype)
    w = _randn((B, S1, N1), g, device, w_dtype, w_scale)
    return IndexerInputs(q, k, w, sparse_count, sparse_mode)


C1 = dict(B=1, S1=256, S2=256, N1=8, N2=1, D=128, sparse_count=64, sparse_mode=3)
C2 = dict(B=1, S1=8192, S2=8192, N1=64, N2=1, D=128, sparse_count=2048, sparse_mode=3, w_scale=1.0 / 8)


@dataclass
class SFAInputs:
    query: torch.Tensor
    key: torch.Tensor
    value: torch.Tensor
    sparse_indices: torch.Tensor
    query_rope: torch.Tensor
    key_rope: torch.Tensor
    scale_value: float
    sparse_block_size: int = 1
    sparse_mode: int = 3
    layout_query: str = "BSND"
    layout_kv: str = "BSND"
    block_table: object = None
    actual_seq_lengths_query: object = None
    actual_seq_lengths_kv: object = None
    block_size: int = 0
    extra: dict = field(default_factory=dict)

    def kwargs(self):
        return dict(scale_value=self.scale_value, block_table=self.block_table,
                    actual_seq_lengths_query=self.actual_seq_lengths_query,
                    actual_seq_lengths_kv=self.actual_seq_lengths_kv,
                    query_rope=self.query_rope, key_rope=self.key_rope,
                    sparse_block_size=self.sparse_block_size, layout_query=self.layout_query,
                    layout_kv=self.layout_kv, sparse_mode=self.sparse_mode,
                    return_softmax_lse=True, block_size=self.block_size)


def causal_block_indices(B, S1, S2, sparse_count, sparse_block_size, sparse_mode, g, device):
    """Reference index generator semantics (test_sfa_triton.py:64-85): for each row,
    ``min(sparse_count, ceil(threshold / bs))`` distinct sorted block ids in
    ``[0, ceil(threshold / bs))``, -1 padded; rows with threshold <= 0 are all -1."""
    s1 = torch.arange(S1, device=device, dtype=torch.int64)
    thr = torch.full_like(s1, S2) if sparse_mode == 0 else (S2 - S1 + s1 + 1)
    nblk = torch.clamp((thr + sparse_block_size - 1) // sparse_block_size, min=0)
    nblk = nblk.repeat(B)
    si = sorted_random_subsets(nblk, sparse_count, g, device,
                               max_pos=max(1, (S2 + sparse_block_size - 1) // sparse_block_size))
    return si.reshape(B, S1, 1, sparse_count)


def sfa_prefill_inputs(B=1, S1=4096, S2=4096, N1=128, D=512, Dr=64, sparse_count=2048,
                       sparse_block_size=1, sparse_mode=3, dtype=torch.bfloat16, device="cpu", seed=42):
    """C3 defaults: BSND MLA-absorb prefill, value = key."""
    g = _gen(device, seed)
    q = _randn((B, S1, N1, D), g, device, dtype)
    k = _randn((B, S2, 1, D), g, device, dtype)
    qr = _randn((B, S1, N1, Dr), g, device, dtype)
    kr = _randn((B, S2, 1, Dr), g, device, dtype)
    gi = _gen(device, seed + 1000)
    si = causal_block_indices(B, S1, S2, sparse_count, sparse_block_size, sparse_mode, gi, device)
    return SFAInputs(q, k, k, si, qr, kr, 1.0 / math.sqrt(D + Dr), sparse_block_size, sparse_mode)


def sfa_decode_inputs(B=64, N1=128, D=512, Dr=64, block_size=128, len_lo=4096, len_hi=32768,
                      sparse_count=2048, dtype=torch.bfloat16, device="cpu", seed=42):
    """C4 defaults: PA_BSND decode, one query token per batch, per-batch kv lengths
    uniform in [len_lo, len_hi], block table a random permutation of a pool sized to the
    total tokens (padded with -1), ``sparse_count`` distinct sorted positions below each length."""
    g = _gen(device, seed)
    gi = _gen("cpu", seed + 1000)
    lens = torch.randint(len_lo, len_hi + 1, (B,), generator=gi, dtype=torch.int64)
    nb = (lens + block_size - 1) // block_size
    pool = int(nb.sum().item())
    maxb = int(nb.max().item())
    perm = torch.randperm(pool, generator=gi).to(torch.int32)
    bt = torch.full((B, maxb), -1, dtype=torch.int32)
    off = 0
    for b in range(B):
        n = int(nb[b])
        bt[b, :n] = perm[off:off + n]
        off += n
    q = _randn((B, 1, N1, D), g, device, dtype)
    qr = _randn((B, 1, N1, Dr), g, device, dtype)
    kc = _randn((pool, block_size, 1, D), g, device, dtype)
    krc = _randn((pool, block_size, 1, Dr), g, device, dtype)
    si = sorted_random_subsets(lens, sparse_count, gi, "cpu").reshape(B, 1, 1, sparse_count)
    return SFAInputs(q, kc, kc, si.to(device), qr, krc, 1.0 / math.sqrt(D + Dr), 1, 3,
                     "BSND", "PA_BSND", bt.to(device), None, lens.to(torch.int32).tolist(), block_size,
                     extra=dict(lens=lens))


# The reference's SFA backward perf shape (perf_sfa_grad_triton.py:23): B=1, S1=512,
# S2=4096, N1=64, top-k 2048, D=512 (+64 rope), causal, bf16.
GRAD_PERF = dict(B=1, S1=512, S2=4096, N1=64, D=512, sparse_count=2048)


def sfa_grad_inputs(B=1, S1=512, S2=4096, N1=64, D=512, Dr=64, sparse_count=2048, sparse_mode=3,
                    dtype=torch.bfloat16, device="cpu", seed=42):
    """Forward inputs plus a seeded d_out for the backward (value = key)."""
    fwd = sfa_prefill_inputs(B, S1, S2, N1, D, Dr, sparse_count, 1, sparse_mode, dtype, device, seed)
    fwd.extra["d_out"] = _randn((B, S1, N1, D), _gen(device, seed + 7), device, dtype)
    return fwd


C5_LENGTHS = (1024, 3000, 6000, 8192)


def tnd_pipeline_inputs(lengths=C5_LENGTHS, N_idx=64, D_idx=128, N1=128, D=512, Dr=64,
                        sparse_count=2048, dtype=torch.bfloat16, device="cpu", seed=42):
    """C5: packed TND sequences; the indexer's top-k feeds SFA in the same run."""
    g = _gen(device, seed)
    T = int(sum(lengths))
    cu = torch.tensor(list(torch.cumsum(torch.tensor(lengths), 0).tolist()), dtype=torch.int32)
    iq = _randn((T, N_idx, D_idx), g, device, dtype)
    ik = _randn((T, 1, D_idx), g, device, dtype)
    iw = _randn((T, N_idx), g, device, torch.float32, 1.0 / 8)
    q = _randn((T, N1, D), g, device, dtype)
    k = _randn((T, 1, D), g, device, dtype)
    qr = _randn((T, N1, Dr), g, device, dtype)
    kr = _randn((T, 1, Dr), g, device, dtype)
    return dict(index_query=iq, index_key=ik, index_weights=iw, query=q, key=k, query_rope=qr,
                key_rope=kr, cu_seqlens=cu, sparse_count=sparse_count, scale_value=1.0 / math.sqrt(D + Dr))
