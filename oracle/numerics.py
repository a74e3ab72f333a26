"""Rounding helpers of the oracle (test infrastructure only).

Restates ``_round_bf16`` / ``_quantize`` of lightning_indexer_numpy.py:20-35 and
``_round_bf16`` of sparse_flash_attention_numpy.py:26-32: fp32 -> 16-bit float
-> fp32 with IEEE round-to-nearest-even. bf16 rounding is the uint32 bias trick
(add 0x7FFF plus the lsb of the kept half, then truncate); fp16 rounding is
numpy's IEEE cast.
"""
import numpy as np


def round_bf16(x):
    """fp32 -> bf16 -> fp32, round to nearest even (lightning_indexer_numpy.py:20-24)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    bias = ((u >> np.uint32(16)) & np.uint32(1)) + np.uint32(0x7FFF)
    return ((u + bias) & np.uint32(0xFFFF0000)).view(np.float32)


def round_fp16(x):
    """fp32 -> fp16 -> fp32 (IEEE RNE; -inf stays -inf)."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def quantize(x, value_dtype):
    """lightning_indexer_numpy.py:27-35: quantise scores to the output dtype."""
    if value_dtype == "fp16":
        return round_fp16(x)
    return round_bf16(x)


def bf16_bits(x):
    """Upper 16 bits of fp32 values that are already bf16-exact."""
    return (np.ascontiguousarray(x, dtype=np.float32).view(np.uint32) >> np.uint32(16)).astype(np.uint16)


def bf16_from_bits(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)
