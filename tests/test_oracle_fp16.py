"""Pins of the oracle's IEEE binary16 conversion (the reference's
__float2half / __half2float, src/voltattn.cu:722-723, 846, 852-853): round to
nearest, ties to even, subnormals, overflow to infinity, checked against
numpy's float16 conversion (an independent IEEE implementation)."""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.filterwarnings("ignore:overflow encountered")


def _edge_values() -> np.ndarray:
    h = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    f = h.view(np.float16).astype(np.float32)
    f = f[np.isfinite(f)]
    # exact ties between neighbouring halves and values just either side
    nxt = np.nextafter(f.astype(np.float16), np.float16(np.inf)).astype(np.float32)
    ok = np.isfinite(nxt)
    mid = ((f[ok].astype(np.float64) + nxt[ok].astype(np.float64)) / 2).astype(np.float32)
    return np.concatenate([f, mid, np.nextafter(mid, np.float32(np.inf)),
                           np.nextafter(mid, np.float32(-np.inf))])


def test_f32_to_f16_matches_numpy_on_ties_and_edges():
    x = _edge_values()
    assert np.array_equal(oracle.f32_to_f16(x), x.astype(np.float16).view(np.uint16))


def test_f32_to_f16_matches_numpy_random_scales():
    rng = np.random.default_rng(1)
    for scale in (1.0, 1e-3, 1e-6, 3e-8, 7e4, 6.6e4):
        x = (rng.standard_normal(200_000) * scale).astype(np.float32)
        assert np.array_equal(oracle.f32_to_f16(x), x.astype(np.float16).view(np.uint16)), scale


def test_f32_to_f16_specials():
    x = np.array([0.0, -0.0, np.inf, -np.inf, 65504.0, 65519.99, 65520.0, 1e9, -1e9,
                  2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0000001, 2.0 ** -26], np.float32)
    assert np.array_equal(oracle.f32_to_f16(x), x.astype(np.float16).view(np.uint16))
    nan = oracle.f32_to_f16(np.array([np.nan], np.float32))[0]
    assert (nan & 0x7C00) == 0x7C00 and (nan & 0x3FF) != 0


def test_f16_to_f32_all_patterns():
    h = np.arange(0, 1 << 16, 97, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(ref)]))
