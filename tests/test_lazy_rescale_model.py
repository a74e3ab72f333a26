"""CPU model of sfa_attn_kernel's online softmax with lazy rescaling.

The kernel (csrc/sfa_fwd.hip, softmax_tile) walks a row's tokens in tiles of 32:
the tile max mx moves the exponent reference m_used only when mx > m_used + TAU,
P = exp(s - m_used) is packed to the io dtype before the PV product, O and the row
sum l are fp32 and are rescaled by exp(m_old - m_new) when m_used moves. The model
below restates that loop in numpy (the TAU values are read from the kernel source)
and shows, on rows whose per-tile maxima climb by 15-35 nats:

* every packed P is finite (at most e^TAU) for both io dtypes;
* the normalised output equals float64 softmax attention within the io dtype's
  rounding, and sum_t exp(s - max) is reproduced from (l, m_used, m_true);
* the threshold the kernel used for fp16 before (40 nats) overflows fp16, so the
  check would catch a regression.
"""
import os
import re

import numpy as np
import pytest

from oracle.numerics import round_bf16, round_fp16

SRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                   "dsa_triton_ascend_amd", "csrc", "sfa_fwd.hip")
TILE = 32
FP16_MAX = 65504.0


def kernel_taus():
    """(fp16 TAU, bf16 TAU) as written in lazy_tau<IO>() of the kernel source."""
    with open(SRC) as f:
        m = re.search(r"lazy_tau\(\)\s*\{\s*return IO == IO_F16 \? ([0-9.]+)f : ([0-9.]+)f;", f.read())
    assert m, "lazy_tau<IO>() not found in sfa_fwd.hip"
    return float(m.group(1)), float(m.group(2))


def model_row(s, v, tau, io):
    """One head of one row: scores s [T] (already scaled), values v [T, D].
    Returns (out [D], m_true, sum_t exp(s - m_true), max packed P)."""
    pack = round_fp16 if io == "fp16" else round_bf16
    m_used = -np.inf
    m_true = -np.inf
    l = np.float32(0)
    o = np.zeros(v.shape[1], np.float32)
    pmax = 0.0
    for t0 in range(0, len(s), TILE):
        st = s[t0:t0 + TILE].astype(np.float32)
        mx = np.float32(st.max())
        m_true = max(m_true, mx)
        m_new = mx if mx > m_used + tau else m_used
        alpha = np.float32(1.0) if m_used == -np.inf else np.float32(np.exp(np.float32(m_used - m_new)))
        m_used = m_new
        p = pack(np.exp(st - np.float32(m_used)).astype(np.float32))
        pmax = max(pmax, float(p.max()))
        o = o * alpha + p @ v[t0:t0 + TILE].astype(np.float32)
        l = l * alpha + np.float32(np.exp(st - np.float32(m_used)).sum())
    out = o / l
    ssum = float(l) * float(np.exp(np.float64(m_used) - np.float64(m_true)))
    return out, float(m_true), ssum, pmax


def climbing_row(rng, climbs, T=256, D=64, io="fp16"):
    """Scores of T tokens (8 tiles of 32): N(0,1) background plus one spike per tile
    whose value climbs by the given nats per tile; the last two spikes are 0.5 apart
    so the output mixes two value rows."""
    s = rng.randn(T).astype(np.float32)
    level = 0.0
    ntiles = T // TILE
    for j in range(1, ntiles):
        level += climbs[(j - 1) % len(climbs)]
        s[j * TILE + rng.randint(TILE)] = level
    s[(ntiles - 2) * TILE + 3] = level - 0.5
    pack = round_fp16 if io == "fp16" else round_bf16
    v = pack(rng.randn(T, D).astype(np.float32))
    return s, v


def reference(s, v):
    s64 = s.astype(np.float64)
    m = s64.max()
    e = np.exp(s64 - m)
    return (e / e.sum()) @ v.astype(np.float64), m, e.sum()


@pytest.mark.parametrize("io", ["fp16", "bf16"])
@pytest.mark.parametrize("climbs", [(15.0,), (35.0,), (15.0, 35.0, 22.5), (11.5, 30.0)])
def test_lazy_rescale_bounds_and_result(io, climbs):
    tau = kernel_taus()[0 if io == "fp16" else 1]
    rng = np.random.RandomState(3)
    for _ in range(4):
        s, v = climbing_row(rng, climbs, io=io)
        out, m_true, ssum, pmax = model_row(s, v, tau, io)
        assert np.isfinite(pmax) and pmax <= np.exp(tau) * (1 + 2 ** -7)
        if io == "fp16":
            assert pmax < FP16_MAX
        ref, m, esum = reference(s, v)
        assert np.all(np.isfinite(out))
        np.testing.assert_allclose(out, ref, rtol=1e-2, atol=1e-2)
        assert abs(m_true - m) <= 1e-6 * max(1.0, abs(m))
        assert abs(ssum - esum) <= 1e-4 * esum


def test_fp16_tau_below_overflow():
    tau16, tau_bf16 = kernel_taus()
    assert np.exp(tau16) < FP16_MAX
    assert np.isfinite(np.float32(np.exp(tau_bf16)))


def test_old_fp16_threshold_overflows():
    """Planted: fp16 with the 40-nat threshold packs P = e^15 .. e^35 to fp16, which is
    +inf, and the output is no longer finite."""
    rng = np.random.RandomState(4)
    s, v = climbing_row(rng, (15.0, 35.0), io="fp16")
    with np.errstate(over="ignore", invalid="ignore"):
        out, _, _, pmax = model_row(s, v, 40.0, "fp16")
    assert not np.isfinite(pmax)
    assert not np.all(np.isfinite(out))
