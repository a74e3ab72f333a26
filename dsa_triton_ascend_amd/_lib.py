"""ctypes binding of ``libdsa_mi355x.so`` (the C ABI declared in include/dsa_mi355x.h).

The library is built in-tree by ``dsa_triton_ascend_amd.build``. There is no
fallback: if the library is missing or fails to load, every operator raises.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libdsa_mi355x.so"

DSA_DTYPE_F16 = 0
DSA_DTYPE_BF16 = 1
DSA_DTYPE_F32 = 2
DSA_OK = 0
DSA_ERR_INVALID = -1
DSA_ERR_UNSUPPORTED = -2
DSA_ERR_HIP = -3

# every symbol the header declares, with its ctypes signature
_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_SZ = ctypes.c_size_t
_F = ctypes.c_float
SIGNATURES = {
    "dsa_abi_version": (_I, []),
    "dsa_last_error": (ctypes.c_char_p, []),
    "dsa_li_score": (_I, [_P, _P, _P, _I, _I, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _I,
                          _P, _I64, _P]),
    "dsa_li_topk": (_I, [_P, _I64, _I, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _P, _P]),
    "dsa_li_topk_workspace_bytes": (_SZ, [_I, _I, _I, _I]),
    "dsa_li_topk_ws": (_I, [_P, _I64, _I, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _P, _P, _SZ, _P]),
    "dsa_sfa_workspace_bytes": (_SZ, [_I, _I, _I, _I, _I, _I]),
    "dsa_sfa_workspace_zero_bytes": (_SZ, []),
    "dsa_sfa_fwd": (_I, [_P, _P, _P, _P, _I, _P, _I, _I, _P, _I, _I, _P, _P, _P, _P, _I, _I, _I,
                         _I, _I, _I, _I64, _I, _F, _P, _P, _P, _P, _SZ, _I, _P]),
    "dsa_sfa_fwd_noalloc": (_I, [_P, _P, _P, _P, _I, _P, _I, _I, _P, _I, _I, _P, _P, _P, _P, _I, _I, _I,
                                 _I, _I, _I, _I64, _I, _F, _P, _P, _P, _I, _P]),
    "dsa_li_score_paged": (_I, [_P, _P, _P, _I, _I, _P, _P, _I, _I, _I64, _P, _P, _I, _I, _I, _I, _I, _I, _I,
                                _I, _P, _I64, _P]),
    "dsa_sli_grad_workspace_bytes": (_SZ, [_I, _I, _I, _I, _I]),
    "dsa_sli_grad_kl_loss": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _P, _I, _P, _P, _P, _P, _I, _I, _I, _I,
                                  _I, _I, _I, _I, _F, _P, _P, _P, _P, _P, _SZ, _P]),
    "dsa_dense_li_softmax_lse": (_I, [_P, _P, _P, _I, _I, _P, _P, _I, _I, _I, _I, _I, _P, _P, _P]),
    "dsa_dense_li_grad_workspace_bytes": (_SZ, [_I, _I, _I, _I]),
    "dsa_dense_li_grad_kl_loss": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _P, _P, _P, _P, _P, _P, _I, _I, _I,
                                       _I, _I, _I, _I, _I, _I, _F, _P, _P, _P, _P, _P, _SZ, _P]),
    "dsa_sfa_bwd_workspace_bytes": (_SZ, [_I, _P, _P, _I, _I, _I, _I, _I, _I, _I64]),
    "dsa_sfa_bwd": (_I, [_P, _P, _P, _P, _I, _P, _I, _I, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I,
                         _I, _I64, _I, _F, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P]),
}

_lib = None


class DSAError(RuntimeError):
    """A HIP-side failure reported by the C ABI."""


def load(path: os.PathLike | None = None) -> ctypes.CDLL:
    """Load the library (once) and bind every declared symbol. Raises if absent."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise RuntimeError(
            f"{p} is missing: build the HIP library first "
            "(python -m dsa_triton_ascend_amd.build or __graft_entry__.build())")
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def check(status: int, what: str) -> None:
    if status == DSA_OK:
        return
    msg = load().dsa_last_error().decode(errors="replace")
    if status in (DSA_ERR_INVALID, DSA_ERR_UNSUPPORTED):
        raise ValueError(msg or what)
    raise DSAError(f"{what}: {msg}")
