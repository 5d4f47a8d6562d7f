"""GPU: decode calls from several streams at once, a captured graph replayed
while eager calls run on other streams, and more streams than ticket slots.

Every stream is bound its own fused-merge ticket slot (va_slots.hpp; one per
stream, one per captured stream of a graph), so calls that overlap never share
merge state: each output must equal the single-stream eager result bit for bit
(the kernels are deterministic). Streams beyond the device's 16 slots run the
two-pass form (partials in ws, separate merge kernel), whose outputs are
within two half-ulps of the fused ones and inside the reference's gate.
Finally va_merge_faults must report no merge that gave up."""
import numpy as np
import pytest

import oracle
import voltattn_amd as va
from tests import gpu_util

pytestmark = pytest.mark.gpu

H, L, D, S, G = 8, 3000, 128, 7, 32
FMTS = [va.Fmt.F16M, va.Fmt.Q8M, va.Fmt.Q4M, va.Fmt.Q3M]


class Inputs:
    def __init__(self, fmt):
        self.fmt = fmt
        self.c = gpu_util.case(va.fmt_bits(fmt), H, L, D, G, 0x57E + int(fmt))
        keys = ["kpay", "vpay", "q"] + ([] if va.is_f16(fmt) else ["ksc", "vsc"])
        self.dev = {k: va.DeviceBuffer.from_array(self.c[k]) for k in keys}

    def bufs(self, out, ws):
        d = self.dev
        return va.DeviceBufs(K=d["kpay"].ptr, V=d["vpay"].ptr,
                             scK=d["ksc"].ptr if "ksc" in d else 0, scV=d["vsc"].ptr if "vsc" in d else 0,
                             q=d["q"].ptr, out=out.ptr, ws=ws.ptr)

    def free(self):
        for x in self.dev.values():
            x.free()


class Outs:
    """One out/ws pair per format."""

    def __init__(self):
        self.out = [va.DeviceBuffer(H * D * 2) for _ in FMTS]
        self.ws = [va.DeviceBuffer(va.ws_bytes(H, D, S)) for _ in FMTS]

    def launch(self, inputs, stream):
        for i, x in enumerate(inputs):
            va.launch(x.fmt, x.bufs(self.out[i], self.ws[i]), H, L, D, S, G=G, stream=stream)

    def results(self):
        return [o.download(np.uint16) for o in self.out]

    def clear(self):
        for o in self.out:
            o.zero()

    def free(self):
        for x in self.out + self.ws:
            x.free()


@pytest.fixture(scope="module")
def inputs():
    xs = [Inputs(f) for f in FMTS]
    yield xs
    for x in xs:
        x.free()


def _eager(inputs):
    o = Outs()
    try:
        o.launch(inputs, None)
        va.sync()
        res = o.results()
    finally:
        o.free()
    for x, r in zip(inputs, res):
        ok, _ = oracle.gate(r.view(np.float16).astype(np.float64), x.c["ref"])
        assert ok, x.fmt.label
    return res


def test_concurrent_streams_and_graph_replays(inputs):
    eager = _eager(inputs)
    NS = 5
    streams = [va.Stream() for _ in range(NS)]
    gstream = va.Stream()
    outs = [Outs() for _ in range(NS)]
    gout = Outs()
    try:
        with va.Graph.capture(gstream) as cap:
            gout.launch(inputs, gstream)
        g = cap.graph
        for rep in range(4):
            for o in outs + [gout]:
                o.clear()
            va.sync()
            print(f"streams rep {rep}: {NS} streams x {len(FMTS)} formats + a graph replay", flush=True)
            for i in range(3):                      # interleaved enqueue, no synchronisation
                for st, o in zip(streams, outs):
                    o.launch(inputs, st)
                if i == 1:
                    g.launch(gstream)
            for st in streams + [gstream]:
                st.synchronize()
            for k, o in enumerate(outs + [gout]):
                for f, got, want in zip(FMTS, o.results(), eager):
                    assert np.array_equal(got, want), (rep, k, f.label)
        g.destroy()
        assert va.merge_faults() == 0
    finally:
        for o in outs + [gout]:
            o.free()
        for st in streams + [gstream]:
            st.destroy()


def test_more_streams_than_ticket_slots(inputs):
    eager = _eager(inputs)
    NS = 20                                          # > 16 slots per device
    streams = [va.Stream() for _ in range(NS)]
    outs = [Outs() for _ in range(NS)]
    try:
        print(f"{NS} streams at once", flush=True)
        for _ in range(2):
            for st, o in zip(streams, outs):
                o.launch(inputs, st)
        for st in streams:
            st.synchronize()
        exact = 0
        for o in outs:
            for x, got, want in zip(inputs, o.results(), eager):
                g = got.view(np.float16).astype(np.float32)
                ok, _ = oracle.gate(g.astype(np.float64), x.c["ref"])
                assert ok, x.fmt.label
                w = want.view(np.float16).astype(np.float32)
                assert np.all(np.abs(g - w) <= 2 * gpu_util.half_ulp(x.c["ref"])), x.fmt.label
                exact += int(np.array_equal(got, want))
        assert exact >= 8 * len(FMTS)          # the streams that hold a slot (fused) are exact
        assert va.merge_faults() == 0
    finally:
        for o in outs:
            o.free()
        for st in streams:
            st.destroy()
