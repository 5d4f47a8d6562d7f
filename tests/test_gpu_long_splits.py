"""GPU: one-slot q8+ decode with long splits (4095 to 13109 positions per split:
many tiles per wave), ragged ends, D 64 and both group sizes: the fused output
against the oracle's double reference within the reference's gate and the fp16
rounding bound, and the split-pass partials against the oracle's split algebra
(src/voltattn.cu:804, 651-672)."""
import math

import numpy as np
import pytest

import oracle
import voltattn_amd as va
from tests import gpu_util
from tests.numerics import tight_bound

pytestmark = pytest.mark.gpu

# (H, L, D, S, G): chunk = ceil(L / S)
SHAPES = [(2, 32768, 128, 8, 32),      # chunk 4096
          (2, 32760, 128, 8, 32),      # chunk 4095
          (3, 65541, 128, 5, 64),      # chunk 13109, ragged last split
          (2, 40000, 64, 8, 32),       # D 64
          (1, 70000, 128, 17, 32)]     # last split shorter than one work-group tile


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "H{}-L{}-D{}-S{}-G{}".format(*s))
def test_long_split_decode(shape):
    H, L, D, S, G = shape
    c = gpu_util.case(8, H, L, D, G, 0x10C5 ^ (H * 131 + L * 7 + D + S + G))
    print(f"case q8+ H={H} L={L} D={D} S={S} G={G} chunk={va.split_chunk(L, S)}", flush=True)
    got = gpu_util.run_case(va.Fmt.Q8M, c, S)["out"].reshape(H, D)
    ref = c["ref"].astype(np.float64).reshape(H, D)
    ok, maxerr = oracle.gate(got.ravel(), ref.ravel())
    assert ok, f"reference gate failed, maxerr={maxerr:.3e}"
    bound = tight_bound(ref)
    assert np.all(np.abs(got - ref) <= bound), float(np.max(np.abs(got - ref) / bound))


@pytest.mark.parametrize("shape", SHAPES[:3], ids=lambda s: "H{}-L{}-D{}-S{}-G{}".format(*s))
def test_long_split_partials(shape):
    H, L, D, S, G = shape
    c = gpu_util.case(8, H, L, D, G, 0x20C5 ^ (H * 131 + L * 7 + D + S + G))
    print(f"case q8+ splits H={H} L={L} D={D} S={S} G={G}", flush=True)
    ws = gpu_util.run_case(va.Fmt.Q8M, c, S, splits_only=True)["ws"].astype(np.float64)
    _, lse, avg = oracle.split_attention(c["kd"], c["vd"], c["q"], H, L, D, S)
    for h in range(H):
        for s in range(S):
            m, l, o = ws[h, s, 0], ws[h, s, 1], ws[h, s, 2:]
            assert l > 0.0
            lse2 = m + math.log2(l)
            assert abs(lse2 - lse[h, s] / math.log(2.0)) <= 2e-5 * (1 + abs(lse2)), (h, s)
            np.testing.assert_allclose(o / l, avg[h, s], rtol=2e-5, atol=2e-6)


# Splits of more than one round of the two-phase kernel (8192 positions of K,
# then of V, per round; va_phased.hpp), f16+ and q8+: a ragged last round, a
# round of a single work-group tile (its K and V stages share one register
# pair), and a split whose last round holds one position.
ROUND_SHAPES = [("f16+", 16, 2, 40000, 128, 3, 64),    # chunk 13334: 8192 + 5142
                ("q8+", 8, 2, 65541, 128, 4, 32),      # chunk 16386: 8192 + 8192 + 2
                ("f16+", 16, 1, 16385, 64, 1, 64),     # one split: 8192 + 8192 + 1
                ("q8+", 8, 1, 24577, 128, 1, 64)]      # one split: 3 rounds + 1 position


@pytest.mark.parametrize("shape", ROUND_SHAPES, ids=lambda s: "{}-H{}-L{}-D{}-S{}-G{}".format(s[0], *s[2:]))
def test_multi_round_decode(shape):
    name, bits, H, L, D, S, G = shape
    c = gpu_util.case(bits, H, L, D, G, 0x30C5 ^ (H * 131 + L * 7 + D + S + G))
    print(f"case {name} H={H} L={L} D={D} S={S} G={G} chunk={va.split_chunk(L, S)}", flush=True)
    got = gpu_util.run_case(va.Fmt.parse(name), c, S)["out"].reshape(H, D)
    ref = c["ref"].astype(np.float64).reshape(H, D)
    ok, maxerr = oracle.gate(got.ravel(), ref.ravel())
    assert ok, f"reference gate failed, maxerr={maxerr:.3e}"
    bound = tight_bound(ref)
    assert np.all(np.abs(got - ref) <= bound), float(np.max(np.abs(got - ref) / bound))
