"""GPU quantizer (va_quantize) is bit-exact with the oracle's restatement of the
reference's quantize() (src/voltattn.cu:705-745): packed bytes and fp16 scales
identical for every element, for q8/q4/q3 at G=32 and G=64, on the selftest
draws and on adversarial groups (exact .5 ties, zero groups, tiny and huge
magnitudes)."""
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
