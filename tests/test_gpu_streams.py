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


class Job:
    """One decode call with its own device inputs, enqueued on any stream into a
    caller-provided (out, ws) pair: one-slot (tagged merge), grouped (counted
    merge, matrix-core and vector-ALU forms) or paged (counted merge)."""

    def __init__(self, kind, fmt, seed):
        from tests import batch_util
        self.kind, self.fmt, self.dev = kind, fmt, []
        up = lambda a: self.dev.append(va.DeviceBuffer.from_array(a)) or self.dev[-1].ptr
        D, G = 128, 32
        if kind == "mha":
            self.H, L = 6, 2500
            c = gpu_util.case(va.fmt_bits(fmt), self.H, L, D, G, seed)
            self.S = 5
            self.bufs = dict(K=up(c["kpay"]), V=up(c["vpay"]), scK=up(c["ksc"]) if c["ksc"] is not None else 0,
                             scV=up(c["vsc"]) if c["vsc"] is not None else 0, q=up(c["q"]))
            self.launch_args = (self.H, L, D)
            self.out_heads = self.H
        elif kind == "gqa":
            Hq, Hkv, L = 8, 2, 3000
            kv = batch_util.kv_case(fmt, Hkv, L, D, G, seed)
            q = batch_util.queries(Hq, D, seed + 1)
            self.S = va.pick_splits_gqa(fmt, Hq, Hkv, L, D)
            self.bufs = dict(K=up(kv["kpay"]), V=up(kv["vpay"]),
                             scK=up(kv["ksc"]) if kv["ksc"] is not None else 0,
                             scV=up(kv["vsc"]) if kv["vsc"] is not None else 0, q=up(q))
            self.launch_args = (Hq, Hkv, L, D)
            self.out_heads = Hq
        else:
            pb = batch_util.PagedBatch(fmt, [700, 1500, 64], 8, 2, D, G, 64, seed)
            self.pb = pb
            self.S = va.pick_splits_paged(fmt, pb.shape)
            quant = pb.kspool is not None
            self.bufs = dict(K=up(pb.kpool), V=up(pb.vpool), scK=up(pb.kspool) if quant else 0,
                             scV=up(pb.vspool) if quant else 0, block_table=up(pb.table),
                             seq_lens=up(pb.seq_lens), q=up(pb.q))
            self.out_heads = len(pb.lens) * pb.Hq
        self.D, self.G = D, G

    def out_bytes(self):
        return self.out_heads * self.D * 2

    def ws_bytes(self):
        return va.ws_bytes(self.out_heads, self.D, self.S)

    def launch(self, out, ws, stream):
        if self.kind == "paged":
            b = va.PagedBufs(**self.bufs, out=out.ptr, ws=ws.ptr)
            va.decode_paged(self.fmt, b, self.pb.shape, self.S, stream=stream)
            return
        b = va.DeviceBufs(**self.bufs, out=out.ptr, ws=ws.ptr)
        if self.kind == "mha":
            H, L, D = self.launch_args
            va.launch(self.fmt, b, H, L, D, self.S, G=self.G, stream=stream)
        else:
            Hq, Hkv, L, D = self.launch_args
            va.decode_gqa(self.fmt, b, Hq, Hkv, L, D, S=self.S, G=self.G, stream=stream)

    def free(self):
        for x in self.dev:
            x.free()
        if self.kind == "paged":
            self.pb.free()


def test_mixed_merge_protocols_on_concurrent_streams():
    """One-slot (tagged) and grouped / paged (counted) calls interleaved on four
    streams while a captured graph of all four replays on a fifth: every output
    equals its single-stream result bit for bit, and no merge is lost."""
    jobs = [Job("mha", va.Fmt.Q8M, 0x5A1), Job("gqa", va.Fmt.Q8M, 0x5A2),
            Job("gqa", va.Fmt.F16M, 0x5A3), Job("paged", va.Fmt.Q4M, 0x5A4)]
    assert all(j.S <= 64 for j in jobs)                       # all fused
    NS = 4
    streams = [va.Stream() for _ in range(NS)]
    gstream = va.Stream()
    pairs = {}                                                 # (owner, job) -> (out, ws)

    def bufs(owner, k):
        if (owner, k) not in pairs:
            pairs[(owner, k)] = (va.DeviceBuffer(jobs[k].out_bytes()), va.DeviceBuffer(jobs[k].ws_bytes()))
        return pairs[(owner, k)]

    try:
        eager = []
        for k, j in enumerate(jobs):
            out, ws = bufs("eager", k)
            j.launch(out, ws, None)
            va.sync()
            eager.append(out.download(np.uint16))
        for owner in ["graph"] + list(range(NS)):            # nothing is allocated under capture
            for k in range(len(jobs)):
                bufs(owner, k)
        with va.Graph.capture(gstream) as cap:
            for k, j in enumerate(jobs):
                j.launch(*bufs("graph", k), gstream)
        g = cap.graph
        for rep in range(3):
            for (owner, k), (out, _) in pairs.items():
                if owner != "eager":
                    out.zero()
            va.sync()
            print(f"mixed protocols rep {rep}: {NS} streams x {len(jobs)} jobs + a graph replay", flush=True)
            for i in range(2):
                for si, st in enumerate(streams):
                    for k in range(len(jobs)):
                        kk = (k + si) % len(jobs)                 # different job order per stream
                        jobs[kk].launch(*bufs(si, kk), st)
                if i == 0:
                    g.launch(gstream)
            for st in streams + [gstream]:
                st.synchronize()
            for (owner, k), (out, _) in pairs.items():
                if owner != "eager":
                    assert np.array_equal(out.download(np.uint16), eager[k]), (rep, owner, jobs[k].kind, jobs[k].fmt.label)
        g.destroy()
        assert va.merge_faults() == 0
    finally:
        for out, ws in pairs.values():
            out.free()
            ws.free()
        for st in streams + [gstream]:
            st.destroy()
        for j in jobs:
            j.free()
