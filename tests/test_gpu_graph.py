"""Launch sequences that a serving loop would use: decode steps captured into
a HIP graph and replayed, many consecutive calls (the fused merge's arrival
counters rotate over a fixed set of slots and must reset themselves), and
calls alternating between two streams. Every output must equal the eager,
single-call result bit for bit (the kernels are deterministic)."""
import numpy as np
import pytest

import oracle
import voltattn_amd as va
from tests import gpu_util

pytestmark = pytest.mark.gpu

H, L, D, S, G = 8, 3000, 128, 7, 32
FMTS = [va.Fmt.F16M, va.Fmt.Q8M, va.Fmt.Q4M, va.Fmt.Q3M]


class Staged:
    """One case's inputs resident on the device with its own out/ws."""

    def __init__(self, fmt):
        self.fmt = fmt
        self.c = gpu_util.case(va.fmt_bits(fmt), H, L, D, G, 0x6A6A + int(fmt))
        keys = ["kpay", "vpay", "q"] + ([] if va.is_f16(fmt) else ["ksc", "vsc"])
        self.dev = {k: va.DeviceBuffer.from_array(self.c[k]) for k in keys}
        self.out = va.DeviceBuffer(H * D * 2)
        self.ws = va.DeviceBuffer(va.ws_bytes(H, D, S))
        d = self.dev
        self.b = va.DeviceBufs(K=d["kpay"].ptr, V=d["vpay"].ptr,
                               scK=d["ksc"].ptr if "ksc" in d else 0,
                               scV=d["vsc"].ptr if "vsc" in d else 0,
                               q=d["q"].ptr, out=self.out.ptr, ws=self.ws.ptr)

    def launch(self, stream=None):
        va.launch(self.fmt, self.b, H, L, D, S, G=G, stream=stream)

    def result(self):
        return self.out.download(np.uint16)

    def clear(self):
        self.out.zero()

    def free(self):
        for x in list(self.dev.values()) + [self.out, self.ws]:
            x.free()


@pytest.fixture(scope="module")
def staged():
    st = [Staged(f) for f in FMTS]
    yield st
    for s in st:
        s.free()


def _eager(staged):
    res = []
    for s in staged:
        s.launch()
        va.sync()
        res.append(s.result())
        ok, _ = oracle.gate(res[-1].view(np.float16).astype(np.float64), s.c["ref"])
        assert ok, s.fmt.label
    return res


def test_graph_replays_match_eager(staged):
    eager = _eager(staged)
    stream = va.Stream()
    try:
        with va.Graph.capture(stream) as cap:
            for s in staged:
                s.launch(stream)
        g = cap.graph
        for rep in range(4):
            for s in staged:
                s.clear()
            va.sync()
            g.launch(stream)
            stream.synchronize()
            for s, want in zip(staged, eager):
                assert np.array_equal(s.result(), want), (rep, s.fmt.label)
            staged[rep % len(staged)].launch()          # eager work between replays
            va.sync()
        g.destroy()
    finally:
        stream.destroy()


def test_many_consecutive_calls_reuse_ticket_slots(staged):
    eager = _eager(staged)
    for i in range(40):                                 # > the number of ticket slots
        s = staged[i % len(staged)]
        s.clear()
        s.launch()
        va.sync()
        assert np.array_equal(s.result(), eager[i % len(staged)]), i


def test_two_streams_interleaved(staged):
    eager = _eager(staged)
    s1, s2 = va.Stream(), va.Stream()
    try:
        for s in staged:
            s.clear()
        va.sync()
        for _ in range(3):
            staged[0].launch(s1)
            staged[1].launch(s2)
            staged[2].launch(s1)
            staged[3].launch(s2)
        s1.synchronize()
        s2.synchronize()
        for s, want in zip(staged, eager):
            assert np.array_equal(s.result(), want), s.fmt.label
    finally:
        s1.destroy()
        s2.destroy()
