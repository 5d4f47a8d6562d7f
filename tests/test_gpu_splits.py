"""GPU first pass alone (va_decode_splits): every (head, split) partial
(m, l, o[D]) in the workspace matches the oracle's split algebra
(split_attention: chunk = ceil(L/S), src/voltattn.cu:804) — the split's
log-sum-exp m + log2(l) (log2 units) and its normalised output o/l — and empty
splits carry l = 0, o = 0 with the finite sentinel m, as the reference's
-FLT_MAX convention requires (src/voltattn.cu:142, 109-112). The lazy rescale
may leave m above or below the split's true maximum; these two quantities are
invariant to it."""
import math

import numpy as np
import pytest

import oracle
import voltattn_amd as va
from tests import gpu_util

pytestmark = pytest.mark.gpu

SHAPES = [(8, 257, 128, 3), (2, 4096, 128, 5), (8, 513, 64, 4),   # selftest multi-split shapes
          (4, 9, 128, 4),                                          # last split empty
          (3, 5, 64, 8),                                           # S > L: three empty splits
          (2, 1, 128, 1),                                          # a single position
          (2, 3000, 128, 7)]                                       # ragged splits, partial tiles
FMTS = [va.Fmt.F16, va.Fmt.F16M, va.Fmt.Q8, va.Fmt.Q8M, va.Fmt.Q4, va.Fmt.Q4M, va.Fmt.Q3M]


@pytest.mark.parametrize("fmt", FMTS, ids=lambda f: f.label)
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "H{}-L{}-D{}-S{}".format(*s))
def test_split_partials(fmt, shape):
    H, L, D, S = shape
    G = 32
    c = gpu_util.case(va.fmt_bits(fmt), H, L, D, G, 0x5EED ^ (H * 131 + L * 7 + D + S))
    print(f"case {fmt.label} H={H} L={L} D={D} S={S}", flush=True)
    ws = gpu_util.run_case(fmt, c, S, splits_only=True)["ws"].astype(np.float64)
    _, lse, avg = oracle.split_attention(c["kd"], c["vd"], c["q"], H, L, D, S)
    chunk = va.split_chunk(L, S)
    for h in range(H):
        for s in range(S):
            m, l, o = ws[h, s, 0], ws[h, s, 1], ws[h, s, 2:]
            if min(L, s * chunk) >= min(L, s * chunk + chunk):       # empty split
                assert l == 0.0 and np.all(o == 0.0) and m <= -1e29, (h, s, m, l)
                continue
            assert l > 0.0
            lse2 = m + math.log2(l)
            assert abs(lse2 - lse[h, s] / math.log(2.0)) <= 2e-5 * (1 + abs(lse2)), (h, s)
            np.testing.assert_allclose(o / l, avg[h, s], rtol=2e-5, atol=2e-6)


@pytest.mark.parametrize("fmt", [va.Fmt.F16M, va.Fmt.Q8M, va.Fmt.Q3M], ids=lambda f: f.label)
def test_merge_pass_matches_fused(fmt):
    """va_decode (fused last-group merge) and va_decode_splits + va_merge (separate
    merge kernel) give identical fp16 outputs on the same partials' algebra."""
    H, L, D, S, G = 8, 2000, 128, 6, 32
    c = gpu_util.case(va.fmt_bits(fmt), H, L, D, G, 0xABCD)
    fused = gpu_util.run_case(fmt, c, S)
    ws = va.DeviceBuffer.from_array(gpu_util.run_case(fmt, c, S, splits_only=True)["ws"])
    out = va.DeviceBuffer(H * D * 2)
    try:
        va.merge(ws.ptr, out.ptr, H, D, S)
        va.sync()
        two_pass = out.download(np.uint16).view(np.float16).astype(np.float32)
    finally:
        ws.free()
        out.free()
    ok, _ = oracle.gate(two_pass, c["ref"])
    assert ok
    assert np.all(np.abs(two_pass - fused["out"]) <= 2 * gpu_util.half_ulp(c["ref"]))
