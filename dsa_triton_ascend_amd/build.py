"""Build ``libdsa_mi355x.so`` in-tree with hipcc for gfx950.

``python -m dsa_triton_ascend_amd.build`` compiles every translation unit under
``csrc/`` (in parallel) and links the shared library next to this file. All
HIP code is compiled with packed-fp32 instruction selection disabled.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libdsa_mi355x.so"
OBJ = PKG / "_obj"
ARCH = os.environ.get("DSA_OFFLOAD_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
COMMON = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-Wno-unused-result", "-I", str(PKG.parent / "include")]

SOURCES = ["li_score.hip", "li_topk.hip", "sfa_fwd.hip", "sfa_bwd.hip", "sli_grad.hip", "capi.cpp"]


# Kernels whose float code never relies on NaN propagation: lets fmaxf lower to a
# single v_max_f32 without the IEEE-mode canonicalisation of each operand.
NO_NANS = {"li_score.hip", "sfa_fwd.hip", "sfa_bwd.hip"}


def _compile(src: Path, obj: Path) -> None:
    extra = ["-fno-honor-nans"] if src.name in NO_NANS else []
    cmd = [HIPCC, *COMMON, *extra, "-x", "hip", "-c", str(src), "-o", str(obj)]
    p = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in p.stderr.splitlines() if noise not in l)
    if p.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")


def build(verbose: bool = True) -> Path:
    OBJ.mkdir(exist_ok=True)
    objs = []
    with cf.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        futs = []
        for s in SOURCES:
            o = OBJ / (Path(s).stem + ".o")
            objs.append(o)
            futs.append(ex.submit(_compile, CSRC / s, o))
        for f in futs:
            f.result()
    tmp = LIB.with_suffix(".so.tmp")
    # hipBLASLt (the SFA backward's dense d_key / d_value products) is loaded with dlopen on
    # the first backward call, so it is not a load-time dependency of the library
    cmd = [HIPCC, "-shared", f"--offload-arch={ARCH}", "-o", str(tmp), *map(str, objs), "-ldl"]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"link failed:\n{p.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()
