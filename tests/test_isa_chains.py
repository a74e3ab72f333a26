"""The SFA forward's S^T chains are inline-asm MFMAs with VGPR accumulators
(dsa_common.hpp: mfma32_vacc*). The compiler does not know those MFMAs are in flight,
so it could copy or reuse an accumulator register between two steps of a chain (or
before its drain) and read a result that is not there yet: a silent wrong answer that a
GPU test sees only on the shapes where the register allocation happens to do it.

This test compiles csrc/sfa_fwd.hip for gfx950 (device code only, as assembly) and walks
every chain along the control flow: from its first MFMA (src C = 0) until the drain (at
least 18 wait states of s_nop after a chain MFMA), no other vector instruction on any path
may name an accumulator register. CPU only; needs hipcc."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
SRC = os.path.join(ROOT, "dsa_triton_ascend_amd", "csrc", "sfa_fwd.hip")
DRAIN = 18   # wait states after the last MFMA of a chain (dsa_common.hpp: vacc_drain)

_MFMA = re.compile(r"\s*v_mfma_f32_32x32x16_(?:bf16|f16) v\[(\d+):(\d+)\], (v\[\d+:\d+\]), (v\[\d+:\d+\]), (\S+)")


def _regs(text):
    out = set()
    for a, b in re.findall(r"v\[(\d+):(\d+)\]", text):
        out |= set(range(int(a), int(b) + 1))
    for a in re.findall(r"(?<![\w\[:])v(\d+)\b", text):
        out.add(int(a))
    return out


def chain_violations(lines):
    """(number of asm chains, list of (line number, instruction)) for an ISA listing."""
    labels = {}
    for i, line in enumerate(lines):
        m = re.match(r"^(\.?\w+):", line)
        if m:
            labels[m.group(1)] = i
    bad, chains = [], 0
    for i, line in enumerate(lines):
        m = _MFMA.match(line)
        if not (m and m.group(5) == "0"):
            continue
        if not any("ASMSTART" in lines[k] for k in range(max(0, i - 3), i)):
            continue   # a compiler-issued MFMA: the compiler tracks its hazards itself
        chains += 1
        stack, seen = [(i + 1, int(m.group(1)), int(m.group(2)), 0)], set()
        while stack:
            j, lo, hi, nops = stack.pop()
            while j < len(lines):
                key = (j, lo, hi, nops)
                if key in seen:
                    break
                seen.add(key)
                raw = lines[j]
                ins = raw.split(";")[0].strip()
                if not ins or ins.startswith((".", "%")):
                    j += 1
                    continue
                mm = _MFMA.match(raw)
                if mm and mm.group(5) == f"v[{lo}:{hi}]":   # the next step (its result may move)
                    lo, hi, nops = int(mm.group(1)), int(mm.group(2)), 0
                    j += 1
                    continue
                op = ins.split()[0]
                if op == "s_nop":
                    nops += int(ins.split()[1]) + 1
                    if nops >= DRAIN:
                        break
                    j += 1
                    continue
                if not op.startswith("s_") and _regs(ins) & set(range(lo, hi + 1)):
                    if (j + 1, ins) not in bad:
                        bad.append((j + 1, ins))
                    break
                if op == "s_branch":
                    j = labels[ins.split()[1]]
                    continue
                if op.startswith("s_cbranch"):
                    stack.append((labels[ins.split()[1]], lo, hi, nops))
                if op in ("s_endpgm", "s_setpc_b64"):
                    break
                j += 1
    return chains, bad


def test_checker_flags_a_copy_in_flight():
    """The walk itself: a copy of the accumulator before the drain is found, on the
    fall-through path and behind a branch; the same code with the drain first is not."""
    bad_seq = ["\t;;#ASMSTART", "\tv_mfma_f32_32x32x16_bf16 v[2:17], v[20:23], v[24:27], 0", "\t;;#ASMEND",
               "\tv_mfma_f32_32x32x16_bf16 v[2:17], v[20:23], v[28:31], v[2:17]",
               "\ts_cbranch_vccz .LBB0_2", "\ts_nop 3", ".LBB0_2:", "\tv_mov_b32_e32 v40, v5", "\ts_endpgm"]
    assert len(chain_violations(bad_seq)[1]) == 1
    ok_seq = bad_seq[:4] + ["\ts_nop 15", "\ts_nop 1"] + bad_seq[4:]
    assert chain_violations(ok_seq) == (1, [])


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
def test_sfa_forward_chains_never_touched_in_flight(tmp_path):
    asm = tmp_path / "sfa_fwd.s"
    cmd = [HIPCC, "-O3", "-std=c++17", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "-Wno-unused-result", "-I", os.path.join(ROOT, "include"), "-fno-honor-nans",
           "-x", "hip", "-S", "--cuda-device-only", SRC, "-o", str(asm)]
    p = subprocess.run(cmd, capture_output=True, text=True)
    assert p.returncode == 0, p.stderr[-2000:]
    chains, bad = chain_violations(asm.read_text().splitlines())
    assert chains >= 24, f"expected the S^T chains of every attention instantiation, found {chains}"
    assert not bad, f"accumulator touched while its chain is in flight: {bad[:5]}"
