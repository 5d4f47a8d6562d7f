"""Child process of tests/test_zz_no_alloc.py::test_noalloc_workspace_has_one_owner.

Runs in a fresh process, so no earlier test holds a ticket slot or the
allocation-free workspace. With every ticket slot bound by captured graphs,
va_decode_noalloc takes the two-pass form, which uses the device's one
workspace: it must be bound to one owner at a time, refuse (VA_EBUSY) a call
from another owner while the owner's work may still run, move to a new owner
once the old one is idle (eager streams) or released (per-thread streams,
captures), and never give a corrupted output. Prints "noalloc child: ok"."""
from __future__ import annotations

import ctypes as C
import sys
import threading
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))

import numpy as np  # noqa: E402

import oracle  # noqa: E402
import voltattn_amd as va  # noqa: E402
from tests import gpu_util  # noqa: E402

VA_EBUSY = 8
PER_THREAD = 2                  # hipStreamPerThread
FMT, D, G = va.Fmt.Q8M, 128, 32


class Case:
    def __init__(self, H, L, S, seed):
        self.c = gpu_util.case(8, H, L, D, G, seed)
        self.H, self.L, self.S = H, L, S
        c = self.c
        self.bufs = [va.DeviceBuffer.from_array(c[k]) for k in ("kpay", "vpay", "ksc", "vsc", "q")]
        self.out = va.DeviceBuffer(H * D * 2)
        self.ws = va.DeviceBuffer(va.ws_bytes(H, D, S))

    def bufs_c(self, ws=True):
        k, v, sk, sv, q = self.bufs
        return va.DeviceBufs(K=k.ptr, V=v.ptr, scK=sk.ptr, scV=sv.ptr, q=q.ptr, out=self.out.ptr,
                             ws=self.ws.ptr if ws else 0)._c()

    def decode(self, stream):
        cb = self.bufs_c()
        return va.lib.va_decode(int(FMT), C.byref(cb), self.H, self.L, D, G, self.S, stream)

    def two_pass(self, stream):
        """The two-pass form's kernels run explicitly: partials to ws, then the merge."""
        cb = self.bufs_c()
        va.check(va.lib.va_decode_splits(int(FMT), C.byref(cb), self.H, self.L, D, G, self.S, stream))
        va.check(va.lib.va_merge(self.ws.ptr, self.out.ptr, self.H, D, self.S, stream))

    def noalloc(self, stream):
        cb = self.bufs_c(ws=False)
        return va.lib.va_decode_noalloc(int(FMT), C.byref(cb), self.H, self.L, D, G, self.S, stream)

    def result(self):
        return self.out.download(np.uint16)

    def check(self, want, what):
        got = self.result()
        assert np.array_equal(got, want), what
        ok, maxerr = oracle.gate(got.view(np.float16).astype(np.float64), self.c["ref"])
        assert ok, (what, maxerr)


def step(msg):
    print(f"noalloc child: {msg}", flush=True)


def main():
    ref_stream = va.Stream()
    A, B = Case(16, 3000, 8, 0xB1), Case(8, 2000, 6, 0xB2)
    small = [Case(4, 257, 3, 0xC0 + i) for i in range(16)]
    # references: the fused form (graphs) and the two-pass form (everything the
    # workspace serves, and the per-thread default stream)
    want = {}
    for name, x in [(f"g{i}", s) for i, s in enumerate(small)]:
        va.check(x.decode(ref_stream.handle))
        ref_stream.synchronize()
        want[name] = x.result()
        x.out.zero()
    for name, x in (("A", A), ("B", B)):
        x.two_pass(ref_stream.handle)
        ref_stream.synchronize()
        want[name] = x.result()
        x.out.zero()
    step("references done")

    # every ticket slot bound by a captured graph (the reference stream's idle
    # slot is taken over by one of them)
    gstreams = [va.Stream() for _ in range(16)]
    graphs = []
    for st, s in zip(gstreams, small):
        with va.Graph.capture(st) as cap:
            va.check(s.decode(st.handle))
        graphs.append(cap.graph)
    step("16 graphs captured")

    # X: busy for ~1 ms (a 2 GiB fill) ahead of its two-pass call, which binds the workspace
    X, Y = va.Stream(), va.Stream()
    big = va.DeviceBuffer(2 << 30)
    va.fill_normal(big.ptr, (2 << 30) // 4, 7, X)
    assert A.noalloc(X.handle) == 0, va.lib.va_last_error()
    rc = B.noalloc(Y.handle)                         # X's work may still run: refused
    assert rc == VA_EBUSY, (rc, va.lib.va_last_error())
    assert b"bound to another" in va.lib.va_last_error()
    X.synchronize()
    A.check(want["A"], "A on X")
    assert B.noalloc(Y.handle) == 0, va.lib.va_last_error()     # X idle: the binding moves to Y
    Y.synchronize()
    B.check(want["B"], "B on Y")
    step("eager streams: refused while busy, moved once idle, outputs exact")

    # per-thread default streams: va_decode's two-pass form per thread; the
    # workspace is bound per thread and freed by va_stream_release
    errs = []
    order = threading.Barrier(2)

    def worker(i, x):
        try:
            va.check(x.decode(PER_THREAD))
            va.check(va.lib.va_stream_sync(PER_THREAD))
            x.check(want["A" if i == 0 else "B"], f"per-thread decode {i}")
            if i == 0:
                assert x.noalloc(PER_THREAD) == 0, va.lib.va_last_error()   # Y is idle: moves here
                va.check(va.lib.va_stream_sync(PER_THREAD))
            order.wait()
            if i == 1:
                assert x.noalloc(PER_THREAD) == VA_EBUSY                  # thread 0 holds it
            order.wait()
            if i == 0:
                va.check(va.lib.va_stream_release(PER_THREAD))
            order.wait()
            if i == 1:
                assert x.noalloc(PER_THREAD) == 0, va.lib.va_last_error()
                va.check(va.lib.va_stream_sync(PER_THREAD))
                x.check(want["B"], "per-thread noalloc")
                va.check(va.lib.va_stream_release(PER_THREAD))
        except BaseException as e:                      # reported by the main thread
            errs.append(e)
            order.abort()

    th = [threading.Thread(target=worker, args=(0, A)), threading.Thread(target=worker, args=(1, B))]
    for t in th:
        t.start()
    for t in th:
        t.join()
    if errs:
        raise errs[0]
    step("per-thread streams: bound per thread, released, outputs exact")

    # a capture takes the free workspace; eager callers are refused until the graph is destroyed
    Z = va.Stream()
    A.out.zero()
    with va.Graph.capture(Z) as cap:
        assert A.noalloc(Z.handle) == 0, va.lib.va_last_error()
    gz = cap.graph
    for _ in range(2):
        gz.launch(Z)
        Z.synchronize()
        A.check(want["A"], "A in a graph")
        A.out.zero()
    assert B.noalloc(Y.handle) == VA_EBUSY
    gz.destroy()
    assert B.noalloc(Y.handle) == 0, va.lib.va_last_error()
    Y.synchronize()
    B.check(want["B"], "B after the graph")
    step("capture: holds the workspace until destroyed")

    for g, st, s, i in zip(graphs, gstreams, small, range(16)):
        s.out.zero()
        g.launch(st)
        st.synchronize()
        s.check(want[f"g{i}"], f"graph {i}")
        g.destroy()
    assert va.merge_faults() == 0
    for st in gstreams + [X, Y, Z, ref_stream]:
        st.destroy()
    big.free()
    print("noalloc child: ok", flush=True)


if __name__ == "__main__":
    main()
