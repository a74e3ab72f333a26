"""Host-side helpers shared by the two operators: length normalisation,
dtype codes, stream handles and the small int32 index arrays the C ABI takes."""
from __future__ import annotations

import torch

from . import _lib

INT64_MAX = 9223372036854775807


def dtype_code(dt: torch.dtype, what: str, allow_f32: bool = False) -> int:
    if dt == torch.bfloat16:
        return _lib.DSA_DTYPE_BF16
    if dt == torch.float16:
        return _lib.DSA_DTYPE_F16
    if allow_f32 and dt == torch.float32:
        return _lib.DSA_DTYPE_F32
    raise ValueError(f"{what} dtype {dt} not supported (fp16/bf16{'/fp32' if allow_f32 else ''})")


def host_lengths(x, n: int | None = None, default: int | None = None) -> list[int]:
    """None -> [default]*n; list/tuple/ndarray/tensor -> list of ints (a device
    tensor is synchronised to the host, as the reference's .asnumpy() does)."""
    if x is None:
        return [int(default)] * int(n)
    if isinstance(x, torch.Tensor):
        return [int(v) for v in x.detach().to("cpu").reshape(-1).tolist()]
    return [int(v) for v in x]


def batch_lengths(x, n: int, default: int, name: str) -> list[int]:
    """host_lengths(x, n, default) as exactly n per-batch lengths: the kernels read one
    length per batch. A single value applies to every batch, as the reference's
    broadcast `zeros[B] + lengths` does (dense_loss_backward_triton.py:37-43,
    sparse_lightning_indexer_grad_kl_loss_triton.py:308-315); any other count raises."""
    v = host_lengths(x, n, default)
    if len(v) == 1 and n > 1:
        v = v * n
    if len(v) != n:
        raise ValueError(f"{name} must hold {n} per-batch lengths, got {len(v)}")
    return v


def per_batch_from_cumsum(cu: list[int]) -> list[int]:
    """TND cumulative actual_seq_lengths -> per-batch lengths
    (lightning_indexer_triton.py:294-296)."""
    out, prev = [], 0
    for c in cu:
        out.append(c - prev)
        prev = c
    return out


def prefix(lengths: list[int]) -> list[int]:
    out, acc = [0], 0
    for v in lengths:
        acc += v
        out.append(acc)
    return out


def require_device(*tensors: torch.Tensor) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
            raise ValueError("inputs must be torch tensors on the GPU (HIP device)")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError("all inputs must live on the same GPU")
    return dev


def i32(values: list[int], device: torch.device) -> torch.Tensor:
    return torch.tensor(values, dtype=torch.int32).to(device, non_blocking=True)


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
