"""CPU: the V accumulation with a bulk offset fix keeps the signed sum's precision.

The tiled decode kernels (voltattn_amd/csrc/va_tiled.hpp, va_codec.hpp) unpack a
V code as the fp16 subnormal of its stored unsigned value c = v + OFF (OFF = 128,
8, 4 for q8, q4, q3), accumulate o += ev * c per row with one correctly rounded
fp32 fma, sum the weights S = sum(ev) per lane, and add S * (-OFF) to o once
per window of at most 16 rows per lane. The reference accumulates the signed
value directly (src/voltattn.cu:555-557, 640-647: o = o*c + ev*(code - off)).

This emulates both in float32 (products exact, one rounding per add, as
v_fma_mix_f32 does) on softmax-like weights and checks, against the exact sum:

* with the kernel's window the error stays at the signed accumulation's level
  (a few fp32 ulps of sum|ev*v|);
* fixing only once at the end (a whole split as the window) loses several bits
  for q8, whose offset dwarfs typical |v| -- the reason for the window.
"""
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent


def _window_rows():
    """Rows per lane between offset fixes in the product (va_tiled.hpp FIXP)."""
    t = (ROOT / "voltattn_amd" / "csrc" / "va_tiled.hpp").read_text()
    m = re.search(r"constexpr int FIXP = C::VFIX && 2 \* U < (\d+) \? (\d+) / \(2 \* U\) : 1;", t)
    assert m, "FIXP rule not found"
    assert m.group(1) == m.group(2)
    return int(m.group(1))


def _codes(fmt, n, rng):
    if fmt == "q8":   # N(0,1) draws quantized with scale max|x|/127: |v| mostly ~30
        return np.clip(np.round(rng.standard_normal(n) * 127 / 3.5), -127, 127), 128
    off = {"q4": 8, "q3": 4}[fmt]
    return rng.integers(-off, off, n).astype(np.float64), off


def _accumulate(ev, v, off, window):
    """(signed, windowed-unsigned) fp32 results for one lane's element."""
    f32 = np.float32
    signed = f32(0)
    o, S = f32(0), f32(0)
    u = v + off
    for j in range(len(ev)):
        e = float(ev[j])
        signed = f32(float(signed) + e * v[j])           # fma: exact product, one rounding
        o = f32(float(o) + e * u[j])
        S = f32(S + f32(e))
        if (j + 1) % window == 0 or j == len(ev) - 1:
            o = f32(float(o) - float(S) * off)         # fma(S, -OFF, o)
            S = f32(0)
    return float(signed), float(o)


def _worst(fmt, window, n=2048, trials=6, seed=7):
    rng = np.random.default_rng(seed)
    ws = wu = 0.0
    for _ in range(trials):
        logits = rng.standard_normal(n) * 2.0
        p = np.exp2(logits - logits.max()).astype(np.float32)
        ev = (p * rng.uniform(0.01, 0.03, n).astype(np.float32)).astype(np.float32)
        v, off = _codes(fmt, n, rng)
        exact = float(np.sum(ev.astype(np.float64) * v))
        mag = float(np.sum(np.abs(ev.astype(np.float64) * v)))
        s, u = _accumulate(ev, v, off, window)
        ws, wu = max(ws, abs(s - exact) / mag), max(wu, abs(u - exact) / mag)
    return ws, wu


@pytest.mark.parametrize("fmt", ["q8", "q4", "q3"])
def test_kernel_window_matches_signed_accumulation(fmt):
    w = _window_rows()
    assert w <= 32
    signed, windowed = _worst(fmt, w)
    assert windowed <= 2.0 ** -20, (fmt, windowed)
    assert windowed <= 8 * max(signed, 2.0 ** -24), (fmt, signed, windowed)


def test_one_fix_per_split_loses_bits_for_q8():
    signed, whole = _worst("q8", window=1 << 30)
    _, windowed = _worst("q8", _window_rows())
    assert whole > 16 * windowed and whole > 2.0 ** -19, (signed, whole, windowed)
