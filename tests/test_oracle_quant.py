"""Pins of the oracle's quantizer/packer and dequantizer (reference quantize()
and dq(), src/voltattn.cu:705-767), with G in {32, 64}:

* hand-made known answers where the fp16 scale is exactly 1 (amax == lim), so
  the codes are lrint(x) itself — exact .5 ties must round to even;
* the scale is the fp16 rounding of fp32 amax/lim (numpy float16 reference);
* invariants on random data: |v| <= lim, the amax element maps to +-lim,
  unclamped codes are within half a step of x / scale;
* storage layouts stated by the reference: q4 element e in byte e/2, low
  nibble first, stored v+8; q3 element e at bits 3*(e%8) of 3-byte granule
  e/8, stored v+4 (built independently below from that granule statement);
* dequant = float(scale) * code, exactly.
"""
import numpy as np
import pytest

import oracle

LIM = {8: 127, 4: 7, 3: 3}


def _quant(x, D, G, bits):
    data, scale = oracle.quantize(x, D, G, bits)
    return data, scale, oracle.codes(data, x.size, bits)


@pytest.mark.parametrize("bits", [8, 4, 3])
@pytest.mark.parametrize("G", [32, 64])
def test_ties_round_to_even_at_unit_scale(bits, G):
    lim = LIM[bits]
    D = 128
    x = np.zeros((1, D), np.float32)
    base = np.array([-lim + 0.5 + k for k in range(2 * lim)], np.float32)  # all .5 ties in range
    for g in range(D // G):
        grp = np.resize(base, G).astype(np.float32)
        grp[0] = lim                                                      # amax = lim -> scale 1
        x[0, g * G:(g + 1) * G] = grp
    data, scale, codes = _quant(x.ravel(), D, G, bits)
    assert np.all(scale == 0x3C00)                                        # fp16 1.0
    assert np.array_equal(codes, np.rint(x.ravel()).astype(np.int32))     # rint: ties to even


@pytest.mark.parametrize("bits", [8, 4, 3])
def test_zero_group_scale_one_codes_zero(bits):
    x = np.zeros(128, np.float32)
    data, scale, codes = _quant(x, 128, 32, bits)
    assert np.all(scale == 0x3C00) and np.all(codes == 0)


@pytest.mark.parametrize("bits", [8, 4, 3])
@pytest.mark.parametrize("G", [32, 64])
def test_scale_is_fp16_of_amax_over_lim(bits, G):
    rng = np.random.default_rng(bits * 7 + G)
    D = 128
    x = rng.standard_normal((50, D)).astype(np.float32)
    x[3] *= 1e-4
    x[4] *= 300.0
    _, scale, _ = _quant(x.ravel(), D, G, bits)
    amax = np.abs(x.reshape(-1, G)).max(axis=1).astype(np.float32)
    want = (amax / np.float32(LIM[bits])).astype(np.float32).astype(np.float16).view(np.uint16)
    assert np.array_equal(scale, want)


@pytest.mark.parametrize("bits", [8, 4, 3])
@pytest.mark.parametrize("G", [32, 64])
def test_code_invariants(bits, G):
    rng = np.random.default_rng(100 + bits + G)
    D = 128
    x = rng.standard_normal((200, D)).astype(np.float32)
    _, scale, codes = _quant(x.ravel(), D, G, bits)
    lim = LIM[bits]
    assert codes.min() >= -lim and codes.max() <= lim
    sh = scale.view(np.float16).astype(np.float32).repeat(G)
    xf = x.ravel()
    # the largest-magnitude element of every group maps to +-lim
    grp = np.abs(xf.reshape(-1, G))
    idx = np.arange(grp.shape[0]) * G + grp.argmax(axis=1)
    assert np.array_equal(np.abs(codes[idx]), np.full(idx.size, lim))
    # unclamped codes: within half a step of x / scale
    t = xf / sh
    un = np.abs(t) <= lim
    assert np.all(np.abs(t[un] - codes[un]) <= 0.5 + 1e-6)


def test_q4_nibble_layout():
    x = np.zeros(128, np.float32)
    x[0], x[1], x[2], x[3] = 7.0, -7.0, 3.0, -1.0           # amax 7 -> scale 1
    data, _, _ = _quant(x, 128, 32, 4)
    assert data[0] == ((-7 + 8) << 4) | (7 + 8)              # element 0 low nibble, 1 high
    assert data[1] == ((-1 + 8) << 4) | (3 + 8)
    assert np.all(data[2:16] == 0x88)                        # zeros stored as 8


def _q3_granule_pack(codes: np.ndarray) -> np.ndarray:
    """Reference statement: element e -> bits 3*(e%8) of 3-byte granule e/8 (v+4)."""
    out = np.zeros(codes.size * 3 // 8, np.uint8)
    for e, v in enumerate(codes):
        g, k = divmod(e, 8)
        word = int(out[3 * g]) | int(out[3 * g + 1]) << 8 | int(out[3 * g + 2]) << 16
        word |= (int(v) + 4) << (3 * k)
        out[3 * g:3 * g + 3] = [word & 0xFF, (word >> 8) & 0xFF, (word >> 16) & 0xFF]
    return out


@pytest.mark.parametrize("G", [32, 64])
def test_q3_granule_layout(G):
    rng = np.random.default_rng(7)
    x = rng.standard_normal(256).astype(np.float32)
    data, _, codes = _quant(x, 128, G, 3)
    assert np.array_equal(data, _q3_granule_pack(codes))


@pytest.mark.parametrize("bits", [8, 4, 3])
@pytest.mark.parametrize("G", [32, 64])
def test_dequant_is_scale_times_code(bits, G):
    rng = np.random.default_rng(11)
    D = 64
    x = rng.standard_normal((20, D)).astype(np.float32)
    data, scale, codes = _quant(x.ravel(), D, G, bits)
    dq = oracle.dequant(data, scale, 20, D, G, bits)
    want = (scale.view(np.float16).astype(np.float64).repeat(G) * codes).astype(np.float32)
    assert np.array_equal(dq, want)


def test_q8_codes_are_signed_bytes():
    x = np.linspace(-1, 1, 64, dtype=np.float32)
    data, _, codes = _quant(x, 64, 64, 8)
    assert np.array_equal(data.view(np.int8).astype(np.int32), codes)
