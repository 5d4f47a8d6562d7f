"""GPU: the fused merge's ticket slots under mixed use. One-query-slot decodes
(tagged partials) and grouped-query decodes (plain partials behind a stored
count) alternate for more calls than there are ticket slots, so every slot is
reused by both protocols in turn. The kernels merge in a fixed order, so every
call must reproduce the first call's output bit for bit; the first outputs are
also checked against the oracle's double reference."""
import numpy as np
import pytest

import oracle
from oracle import batch
import voltattn_amd as va
from tests import batch_util, gpu_util
from tests.numerics import tight_bound

pytestmark = pytest.mark.gpu

CALLS = 40          # > 16 ticket slots: each slot sees both protocols


class _Step:
    def __init__(self, fmt, Hq, Hkv, L, D, G, S, seed):
        self.fmt, self.Hq, self.Hkv, self.L, self.D, self.G, self.S = fmt, Hq, Hkv, L, D, G, S
        c = batch_util.kv_case(fmt, Hkv, L, D, G, seed)
        q = batch_util.queries(Hq, D, seed + 5)
        self.ref = batch.reference_gqa(c["kd"], c["vd"], q, Hq, Hkv, L, D)
        self.bufs = []
        dev = lambda a: self.bufs.append(va.DeviceBuffer.from_array(a)) or self.bufs[-1].ptr
        self.out = va.DeviceBuffer(Hq * D * 2)
        self.ws = va.DeviceBuffer(va.ws_bytes(Hq, D, S))
        self.bufs += [self.out, self.ws]
        self.b = va.DeviceBufs(K=dev(c["kpay"]), V=dev(c["vpay"]),
                               scK=dev(c["ksc"]) if c["ksc"] is not None else 0,
                               scV=dev(c["vsc"]) if c["vsc"] is not None else 0,
                               q=dev(q), out=self.out.ptr, ws=self.ws.ptr)

    def run(self):
        if self.Hq == self.Hkv:
            va.launch(self.fmt, self.b, self.Hq, self.L, self.D, self.S, G=self.G)
        else:
            va.decode_gqa(self.fmt, self.b, self.Hq, self.Hkv, self.L, self.D, S=self.S, G=self.G)
        va.sync()
        return self.out.download(np.uint16).copy()

    def free(self):
        for x in self.bufs:
            x.free()


@pytest.mark.parametrize("fmt", [va.Fmt.Q8M, va.Fmt.F16M], ids=lambda f: f.label)
def test_alternating_merge_protocols(fmt):
    steps = [_Step(fmt, 8, 8, 3000, 128, 32, 5, 0x51),       # one slot per work-group: tagged
             _Step(fmt, 8, 2, 3000, 128, 32, 6, 0x52),       # four slots: counted
             _Step(fmt, 12, 4, 1500, 64, 32, 3, 0x53)]       # three of four slots, D 64: counted
    try:
        first = [s.run() for s in steps]
        for s, got in zip(steps, first):
            g = got.view(np.float16).astype(np.float32)
            ok, maxerr = oracle.gate(g, s.ref)
            assert ok, maxerr
            assert np.all(np.abs(g - s.ref) <= tight_bound(s.ref))
        print(f"{fmt.label}: {CALLS} alternating calls", flush=True)
        for i in range(CALLS):
            s = steps[i % len(steps)]
            assert np.array_equal(s.run(), first[i % len(steps)]), (i, s.Hq, s.Hkv)
    finally:
        for s in steps:
            s.free()
