"""GPU: splits whose work-group tile count is odd (1, 3, 5 tiles, and ragged last
splits). The decode loops run tiles in register-double-buffered pairs and take an
odd last tile on its own; these shapes pin that path in the one-slot kernels
(va_decode, src/voltattn.cu:803-835), the grouped vector-ALU kernels (f16+,
q3+) and the grouped matrix-core kernels (q8+, q4+) against the oracle, within
the reference's gate and the fp16 rounding bound.

Work-group tiles: 128 positions (one-slot f16+, q8+), 256 (one-slot q4+, q3+;
grouped matrix-core). One-slot chunks are ceil(L / S); grouped chunks are whole
multiples of the kind's largest tile."""
import numpy as np
import pytest

import oracle
from oracle import batch
import voltattn_amd as va
from tests import batch_util, gpu_util
from tests.numerics import tight_bound

pytestmark = pytest.mark.gpu

BITS = {va.Fmt.F16M: 16, va.Fmt.Q8M: 8, va.Fmt.Q4M: 4, va.Fmt.Q3M: 3}

# (L, S): chunks of 75 / 275 / 375 / 575 / 640 positions, last splits ragged
ONE_SLOT = [(300, 4), (1100, 4), (1500, 4), (2300, 4), (1919, 3)]


def _check(got, ref, what):
    assert np.all(np.isfinite(got)), what
    ok, maxerr = oracle.gate(got.ravel(), ref.ravel())
    assert ok, (what, maxerr)
    bad = np.abs(got - ref) > tight_bound(ref)
    assert not bad.any(), (what, int(bad.sum()), float(np.abs(got - ref).max()))


@pytest.mark.parametrize("fmt", list(BITS), ids=lambda f: f.label)
@pytest.mark.parametrize("LS", ONE_SLOT, ids=lambda p: f"L{p[0]}-S{p[1]}")
def test_one_slot_odd_tiles(fmt, LS):
    L, S = LS
    H, D, G = 2, 128, 32
    c = gpu_util.case(BITS[fmt], H, L, D, G, 0x0DD1 ^ (L * 13 + S))
    print(f"case {fmt.label} H={H} L={L} S={S} chunk={va.split_chunk(L, S)}", flush=True)
    got = gpu_util.run_case(fmt, c, S)["out"].reshape(H, D).astype(np.float64)
    _check(got, c["ref"].astype(np.float64).reshape(H, D), (fmt.label, L, S))


# (L, S): for the 256-position matrix-core tile, 3, 5, 4 + 3 and 1 tiles per split
# (1792 over S = 2 is 1024 + 768)
GROUPED = [(768, 1), (1280, 1), (1792, 2), (200, 1)]


@pytest.mark.parametrize("fmt", list(BITS), ids=lambda f: f.label)
@pytest.mark.parametrize("LS", GROUPED, ids=lambda p: f"L{p[0]}-S{p[1]}")
def test_grouped_odd_tiles(fmt, LS):
    L, S = LS
    Hq, Hkv, D, G = 8, 2, 128, 32
    seed = 0x0DD2 ^ (L * 17 + S)
    c = batch_util.kv_case(fmt, Hkv, L, D, G, seed)
    q = batch_util.queries(Hq, D, seed + 5)
    print(f"case gqa {fmt.label} Hq={Hq} Hkv={Hkv} L={L} S={S}", flush=True)
    bufs = []
    try:
        dev = lambda a: bufs.append(va.DeviceBuffer.from_array(a)) or bufs[-1].ptr
        out = va.DeviceBuffer(Hq * D * 2)
        ws = va.DeviceBuffer(va.ws_bytes(Hq, D, S))
        bufs += [out, ws]
        b = va.DeviceBufs(K=dev(c["kpay"]), V=dev(c["vpay"]),
                          scK=dev(c["ksc"]) if c["ksc"] is not None else 0,
                          scV=dev(c["vsc"]) if c["vsc"] is not None else 0,
                          q=dev(q), out=out.ptr, ws=ws.ptr)
        va.decode_gqa(fmt, b, Hq, Hkv, L, D, S=S, G=G)
        va.sync()
        got = out.download(np.uint16).view(np.float16).astype(np.float64)
    finally:
        for x in bufs:
            x.free()
    ref = batch.reference_gqa(c["kd"], c["vd"], q, Hq, Hkv, L, D).astype(np.float64)
    _check(got.reshape(ref.shape), ref, (fmt.label, L, S))
