"""GPU quantizer (va_quantize) is bit-exact with the oracle's restatement of the
reference's quantize() (src/voltattn.cu:705-745): packed bytes and fp16 scales
identical for every element, for q8/q4/q3 at G=32 and G=64, on the selftest
draws and on adversarial groups (exact .5 ties, zero groups, tiny and huge
magnitudes). The device dequantizer (va_dequantize) is bit-exact with the
oracle's restatement of dq() (src/voltattn.cu:747-767) on every byte pattern
(random packed bytes: every code value at every position) under adversarial
fp16 scales (zero, subnormal, largest finite, infinite, NaN, negative), and
dequantize(quantize(x)) is the oracle's dequantization of the quantized x."""
import numpy as np
import pytest

import oracle
import voltattn_amd as va

pytestmark = pytest.mark.gpu


def _gpu_quantize(x: np.ndarray, D: int, G: int, bits: int):
    rows = x.size // D
    with va.DeviceBuffer.from_array(x.astype(np.float32)) as dx, \
            va.DeviceBuffer(oracle.packed_bytes(bits, x.size)) as dp, \
            va.DeviceBuffer(rows * (D // G) * 2) as ds:
        va.quantize(bits, G, dx.ptr, rows, D, dp.ptr, ds.ptr)
        va.sync()
        return dp.download(np.uint8), ds.download(np.uint16)


def _adversarial(rows: int, D: int, bits: int, rng: np.random.Generator) -> np.ndarray:
    lim = {8: 127, 4: 7, 3: 3}[bits]
    x = rng.standard_normal((rows, D)).astype(np.float32)
    x[0] = 0.0                                             # all-zero group -> scale 1
    x[1, :] = (np.arange(D) % (2 * lim) - lim + 0.5).astype(np.float32)  # .5 ties at s = 1
    x[1, 0] = lim                                          # amax = lim -> s = 1 exactly
    x[2] *= 1e-6                                           # tiny values, small scales
    x[3] *= 1e4                                            # large magnitudes
    x[4] = np.where(np.arange(D) % 2 == 0, 1.0, -1.0) * 3.0e-8   # scale rounds to 0: codes 0
    x[5] = rng.standard_normal(D).astype(np.float32) * 1e-5        # fp16-subnormal scales
    return x.ravel()


@pytest.mark.parametrize("G", [32, 64])
@pytest.mark.parametrize("bits", [8, 4, 3])
@pytest.mark.parametrize("shape", oracle.SELFTEST_SHAPES[:5:2])
def test_quantize_selftest_draws(bits, G, shape):
    H, L, D, S = shape
    kx, vx, _ = oracle.draw(oracle.selftest_seed(H, L, D, S), H, L, D)
    for x in (kx, vx):
        data, scale = oracle.quantize(x, D, G, bits)
        gdata, gscale = _gpu_quantize(x, D, G, bits)
        assert np.array_equal(gscale, scale)
        assert np.array_equal(gdata, data)


@pytest.mark.parametrize("bits,G,D", [(b, G, D) for b in (8, 4, 3) for G in (32, 64) for D in (64, 128) if G <= D])
def test_quantize_adversarial(bits, G, D):
    x = _adversarial(64, D, bits, np.random.default_rng(bits * 1000 + G + D))
    data, scale = oracle.quantize(x, D, G, bits)
    gdata, gscale = _gpu_quantize(x, D, G, bits)
    assert np.array_equal(gscale, scale)
    assert np.array_equal(gdata, data)


def _gpu_dequantize(data: np.ndarray, scale: np.ndarray, rows: int, D: int, G: int, bits: int) -> np.ndarray:
    with va.DeviceBuffer.from_array(np.ascontiguousarray(data, np.uint8)) as dp, \
            va.DeviceBuffer.from_array(np.ascontiguousarray(scale, np.uint16)) as ds, \
            va.DeviceBuffer(rows * D * 4) as dx:
        va.dequantize(bits, G, dp.ptr, ds.ptr, rows, D, dx.ptr)
        va.sync()
        return dx.download(np.float32)


def _same_bits(got: np.ndarray, want: np.ndarray) -> bool:
    """Equal bit for bit, NaN payloads aside (both sides NaN at the same places)."""
    gn, wn = np.isnan(got), np.isnan(want)
    return bool(np.array_equal(gn, wn) and np.array_equal(got[~gn].view(np.uint32), want[~wn].view(np.uint32)))


@pytest.mark.parametrize("bits,G,D", [(b, G, D) for b in (8, 4, 3) for G in (32, 64) for D in (64, 128) if G <= D])
def test_dequantize_every_code_and_scale(bits, G, D):
    rng = np.random.default_rng(0xDE00 + bits * 100 + G + D)
    rows = 300                                               # random bytes: every code value occurs
    data = rng.integers(0, 256, oracle.packed_bytes(bits, rows * D), dtype=np.uint8)
    scale = rng.standard_normal(rows * (D // G)).astype(np.float16).view(np.uint16)
    special = np.array([0x0000, 0x8000, 0x0001, 0x83FF, 0x7BFF, 0xFBFF, 0x7C00, 0xFC00, 0x7E00, 0x3C00],
                       np.uint16)                            # +-0, subnormals, max, +-inf, NaN, 1
    scale[:special.size] = special
    want = oracle.dequant(data, scale, rows, D, G, bits)
    got = _gpu_dequantize(data, scale, rows, D, G, bits)
    assert _same_bits(got, want)


@pytest.mark.parametrize("G", [32, 64])
@pytest.mark.parametrize("bits", [8, 4, 3])
def test_dequantize_inverts_quantize(bits, G):
    D, rows = 128, 256
    x = _adversarial(rows, D, bits, np.random.default_rng(0xDE50 + bits + G))
    data, scale = _gpu_quantize(x, D, G, bits)
    got = _gpu_dequantize(data, scale, rows, D, G, bits)
    assert _same_bits(got, oracle.dequant(data, scale, rows, D, G, bits))
    lim = {8: 127, 4: 7, 3: 3}[bits]
    s = np.repeat(scale.view(np.float16).astype(np.float32), G)
    ok = np.isfinite(x) & (np.abs(x) <= s * lim)             # inside the clamp: error <= half a step
    assert np.all(np.abs(got - x)[ok] <= 0.5 * s[ok] * (1 + 1e-6) + 1e-30)
