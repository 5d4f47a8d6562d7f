#!/usr/bin/env python3
"""Benchmark of the fused dequant + decode-attention path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

One "step" is one decode step: one query token attending over L cached
positions for all H=32 heads (D=128), i.e. one va_decode() call (split-L
attention pass + log-sum-exp merge), reading a compressed K/V cache that is
already resident in HBM. The headline workload is BASELINE.json's metric at
H=32 D=128 L=16384 with G=32 scales; `value` is the q8+ (fused INT8) decode
rate in tok/s. Every BASELINE config is measured in the same run (`configs`):
q8/q8+ at L=4096, f16/f16+ at 16384 ([1]), q8+ at 16384 and
65536 ([2]), q4+ at 4096, 16384 and 65536 ([3]), q3+ at 65536 and 262144 ([4]),
each with ms, GB/s, MBU against the probed read ceiling, % of the 8 TB/s peak
and tok/s; `formats` repeats the L=16384 rows by format.

Method (reference bench, src/voltattn.cu:967-1070, re-derived for MI355X):
  * read ceiling: a >= 4 GiB buffer (16x the 256 MB Infinity Cache) read with
    128-bit non-temporal loads, best over launch shapes of two forms, the
    reference's grid-stride read and a chunked read (one contiguous chunk per
    work-group, the shape of a decode split) (va_probe_read);
  * K/V are drawn N(0,1) on the GPU, quantized there (bit-exact quantizer) and
    replicated into enough copies to rotate a >= 2 GiB working set, so the
    MALL cannot serve the stream;
  * settle: each row's buffers are created, then the host waits 500 ms
    (--settle-ms) before any step of it runs: for ~100 ms after the previous
    row's (or a probe's) multi-GiB buffers are freed, steps read 2-3.5 us slow
    (q8+ L=16384: 25.3 against 23.4 us; measured on MI355X, not seen after a
    0.5 s wait);
  * warm-up: untimed steps for >= 50 ms of wall time per row (--warm-ms), so
    the shader clock has ramped from its idle level, then W warm-up steps;
  * timed region: device synchronisation, one untimed lead step (so the start
    event is stamped while the GPU is busy and the host's latency to enqueue
    the first timed step is not counted), then K back-to-back steps between two
    HIP events on the launch stream, then synchronisation -> ms_per_step; plus
    the reference's best-of-K single launch, each behind an untimed lead step;
  * correctness: after timing, every row's output (the last timed step; all
    copies hold the same data) is gated head by head against the oracle's
    double reference over the downloaded packed bytes (the reference gates its
    bench on its selftest, src/voltattn.cu:1075-1076); `checked` is true only
    if every row passes, and the process exits non-zero otherwise;
  * roofline: algorithmic bytes per decode-kernel launch (compressed K+V
    payload + fp16 scales: 2*H*L*(D*b/8 + 2*D/G)) over the fused decode
    kernel's mean launch time (the K back-to-back steps between events: one
    launch per step); the split pass alone (va_decode_splits) beside it;
  * size-matched ceiling per row (va_probe_read_sized): the chunked read of
    exactly that row's bytes per launch, on the decode grid (one or two
    4-wave groups per CU), back to back over the same >= 2 GiB rotation; what
    any kernel reading that many bytes per launch takes, launch gap, ramp and
    tail included. `mbu_sized` = the row's GB/s over that read's GB/s;
  * launch floor (va_probe_launch): us per back-to-back launch of an empty
    kernel with the decode step's grid (reported as launch_floor_us); an
    upper bound on the per-step launch cost, since part of it overlaps a
    running kernel;
  * cpu_baseline: the oracle's double-precision reference attention
    (reference(), src/voltattn.cu:769-794) on the headline shape, timed on
    this host (rank 0, N=1 only); `cpu_configs0` is the same on configs[0]
    (q8, L=4096), at 1 core and at T cores, with nproc and the CPU model.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "tok/s + %MBU vs probed HBM ceiling, f16/q8+/q4+ at H32 D128 L16K"
PEAK_HBM_GBPS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def algo_bytes(fmt, H, L, D, G) -> int:
    import voltattn_amd as va
    return 2 * (va.payload_bytes(fmt, H, L, D) + va.scale_bytes(fmt, H, L, D, G))


class Workload:
    """Rotated copies of one format's K/V cache (+ scales) resident in HBM."""

    def __init__(self, va, fmt, H, L, D, G, min_set_bytes, max_copies, seed=0x1234):
        self.va, self.fmt, self.H, self.L, self.D, self.G = va, fmt, H, L, D, G
        n = H * L * D
        self.pay = va.payload_bytes(fmt, H, L, D)
        self.sc = va.scale_bytes(fmt, H, L, D, G)
        self.copy_bytes = 2 * (self.pay + self.sc)
        self.copies = max(1, min(max_copies, math.ceil(min_set_bytes / self.copy_bytes)))
        al = lambda x: (x + 4095) // 4096 * 4096
        self.pay_al, self.sc_al = al(self.pay), al(max(self.sc, 1))
        self.bufs = []
        self.K = self._alloc(self.pay_al * self.copies)
        self.V = self._alloc(self.pay_al * self.copies)
        self.SK = self._alloc(self.sc_al * self.copies) if self.sc else None
        self.SV = self._alloc(self.sc_al * self.copies) if self.sc else None
        self.q = self._alloc(H * D * 2)
        self.out = self._alloc(H * D * 2)
        # copy 0 from seeded N(0,1) draws, on the device
        x = va.DeviceBuffer(n * 4)
        try:
            bits = va.fmt_bits(fmt)
            for dst, sdst, s in ((self.K, self.SK, seed), (self.V, self.SV, seed + 0x4444)):
                va.fill_normal(x.ptr, n, s)
                if bits == 16:
                    va.f32_to_f16(x.ptr, n, dst.ptr)
                else:
                    va.quantize(bits, G, x.ptr, H * L, D, dst.ptr, sdst.ptr)
            va.fill_normal(x.ptr, H * D, seed + 0x8888)
            va.f32_to_f16(x.ptr, H * D, self.q.ptr)
            va.sync()
        finally:
            x.free()
        for c in range(1, self.copies):
            va.check(va.lib.va_memcpy_d2d(self.K.ptr + c * self.pay_al, self.K.ptr, self.pay, None))
            va.check(va.lib.va_memcpy_d2d(self.V.ptr + c * self.pay_al, self.V.ptr, self.pay, None))
            if self.sc:
                va.check(va.lib.va_memcpy_d2d(self.SK.ptr + c * self.sc_al, self.SK.ptr, self.sc, None))
                va.check(va.lib.va_memcpy_d2d(self.SV.ptr + c * self.sc_al, self.SV.ptr, self.sc, None))
        va.sync()
        self.ws = None
        self.S = None

    def _alloc(self, nbytes):
        b = self.va.DeviceBuffer(nbytes)
        self.bufs.append(b)
        return b

    def set_splits(self, S):
        if self.ws is not None:
            self.ws.free()
            self.bufs.remove(self.ws)
        self.S = S
        self.ws = self._alloc(self.va.ws_bytes(self.H, self.D, S))

    def bufs_for(self, c):
        va = self.va
        return va.DeviceBufs(K=self.K.ptr + c * self.pay_al, V=self.V.ptr + c * self.pay_al,
                             scK=self.SK.ptr + c * self.sc_al if self.sc else 0,
                             scV=self.SV.ptr + c * self.sc_al if self.sc else 0,
                             q=self.q.ptr, out=self.out.ptr, ws=self.ws.ptr)

    def free(self):
        for b in self.bufs:
            b.free()
        self.bufs = []


def time_workload(va, w: Workload, steps: int, warmup: int, stream, steps_only: bool = False,
                  warm_ms: float = 50.0) -> dict:
    H, L, D, G, S, fmt = w.H, w.L, w.D, w.G, w.S, w.fmt
    bufs = [w.bufs_for(c) for c in range(w.copies)]
    launch = lambda c: va.launch(fmt, bufs[c % w.copies], H, L, D, S, G=G, stream=stream)
    first = lambda c: va.decode_splits(fmt, bufs[c % w.copies], H, L, D, S, G=G, stream=stream)
    e0, e1 = va.Event(), va.Event()
    try:
        settle()
        # Residency pass: one untimed step on every rotated copy, so every timed
        # step finds its copy's address translations as warm as the others'
        # (first-touch page walks otherwise land in the first lap of the
        # rotation). The data itself still streams from HBM: the rotated set
        # is >= 2 GiB against a 256 MB MALL.
        for c in range(w.copies):
            launch(c)
        # Clock warm-up: untimed steps for >= warm_ms of wall time, so the
        # shader clock has left its idle level (MI355X idles near 100 MHz and
        # ramps over tens of ms; a VALU-bound row timed cold measured 25-30 %
        # slower), then the W warm-up steps.
        t_end = time.perf_counter() + warm_ms / 1e3
        i = 0
        while time.perf_counter() < t_end:
            launch(i)
            i += 1
            if i % 32 == 0:
                va.sync()
        for i in range(warmup):
            launch(i)
        va.sync()
        # (1) the contract's timed region: K back-to-back steps, rotating copies,
        # between two events on the launch stream. One untimed lead step goes
        # first, so the start event is stamped while the GPU is busy and the
        # host's latency to enqueue the first timed step is not counted.
        launch(steps)
        e0.record(stream)
        for i in range(steps):
            launch(i)
        e1.record(stream)
        e1.synchronize()
        va.sync()
        mean_ms = e0.elapsed_ms(e1) / steps
        if steps_only:            # profiling runs: only fused steps of this shape are dispatched
            return {"mean_ms": mean_ms, "best_ms": float("nan"), "kernel_ms": float("nan")}
        # (2) reference method: best single launch, each behind an untimed lead launch
        best_ms = float("inf")
        for i in range(steps):
            launch(2 * i + 1)
            e0.record(stream)
            launch(2 * i + 2)
            e1.record(stream)
            e1.synchronize()
            best_ms = min(best_ms, e0.elapsed_ms(e1))
        # (3) first pass alone, back-to-back: the split pass's mean launch time
        first(steps)
        e0.record(stream)
        for i in range(steps):
            first(i)
        e1.record(stream)
        e1.synchronize()
        kern_ms = e0.elapsed_ms(e1) / steps
        # the output checked below is that of one full step
        launch(0)
        va.sync()
    finally:
        e0.destroy()
        e1.destroy()
    return {"mean_ms": mean_ms, "best_ms": best_ms, "kernel_ms": kern_ms}


def check_workload(va, w: Workload, heads) -> dict:
    """Checker (not timed): the last step's fp16 output against the oracle's
    double reference attention over copy 0's packed bytes (all copies are
    equal), head by head: the reference's gate |got-ref| <= 3e-3 + 2e-2|ref|
    (src/voltattn.cu:903) and the fp16 rounding bound of tests/numerics.py."""
    import numpy as np
    import oracle
    from tests.numerics import tight_bound
    H, L, D, G, fmt = w.H, w.L, w.D, w.G, w.fmt
    bits = va.fmt_bits(fmt)
    out = w.out.download(np.uint16).view(np.float16).astype(np.float64).reshape(H, D)
    q = w.q.download(np.uint16).reshape(H, D)
    row = w.pay // (H * L)
    ns = L * D // G
    worst, ok = 0.0, bool(np.all(np.isfinite(out)))
    for h in heads:
        kp = w.K.download(np.uint8, L * row, offset=h * L * row)
        vp = w.V.download(np.uint8, L * row, offset=h * L * row)
        if bits == 16:
            kd, vd = kp.view(np.float16).astype(np.float32), vp.view(np.float16).astype(np.float32)
        else:
            kd = oracle.dequant(kp, w.SK.download(np.uint16, ns, offset=h * ns * 2), L, D, G, bits)
            vd = oracle.dequant(vp, w.SV.download(np.uint16, ns, offset=h * ns * 2), L, D, G, bits)
        ref = oracle.reference(kd, vd, q[h], 1, L, D).astype(np.float64)
        gate_ok, maxerr = oracle.gate(out[h], ref)
        ok = ok and gate_ok and bool(np.all(np.abs(out[h] - ref) <= tight_bound(ref)))
        worst = max(worst, maxerr)
    return {"checked": ok, "check_heads": list(heads), "check_maxerr": worst}


SETTLE_MS = 500.0     # --settle-ms

# The reference-shape kernel each "+" format runs (va_decode.hip: VA_<KIND>_PHASED).
HEADLINE_KERNEL = {"f16+": "decode_phased", "q8+": "decode_phased", "q4+": "decode_tiled", "q3+": "decode_tiled"}


def settle() -> None:
    """Wait SETTLE_MS after a row's buffers are created (and earlier buffers
    freed) before its first step: steps launched within ~100 ms of freeing a
    multi-GiB buffer measured 2-3.5 us slow on MI355X."""
    time.sleep(SETTLE_MS / 1e3)


def time_fn(va, fn, copies: int, steps: int, warmup: int, stream) -> float:
    """Mean ms of `steps` back-to-back calls fn(copy, stream), rotating copies."""
    e0, e1 = va.Event(), va.Event()
    try:
        settle()
        for c in range(copies):
            fn(c, stream)
        t_end = time.perf_counter() + 0.05  # clock warm-up, as in time_workload
        i = 0
        while time.perf_counter() < t_end:
            fn(i % copies, stream)
            i += 1
            if i % 32 == 0:
                va.sync()
        for i in range(warmup):
            fn(i % copies, stream)
        va.sync()
        fn(steps % copies, stream)          # untimed lead step: the start event is stamped while busy
        e0.record(stream)
        for i in range(steps):
            fn(i % copies, stream)
        e1.record(stream)
        e1.synchronize()
        va.sync()
        return e0.elapsed_ms(e1) / steps
    finally:
        e0.destroy()
        e1.destroy()


def bench_gqa(va, fmt, Hq, Hkv, L, D, G, steps, warmup, stream, min_set) -> dict:
    """Grouped-query decode of one sequence (va_decode_gqa) over rotated KV copies."""
    w = Workload(va, fmt, Hkv, L, D, G, min_set, 256)
    try:
        S = va.pick_splits_gqa(fmt, Hq, Hkv, L, D)
        w.set_splits(S)
        q = w._alloc(Hq * D * 2)
        out = w._alloc(Hq * D * 2)
        ws = w._alloc(va.ws_bytes(Hq, D, S))
        x = w._alloc(Hq * D * 4)
        va.fill_normal(x.ptr, Hq * D, 0x9999)
        va.f32_to_f16(x.ptr, Hq * D, q.ptr)
        va.sync()
        bl = []
        for c in range(w.copies):
            b = w.bufs_for(c)
            b.q, b.out, b.ws = q.ptr, out.ptr, ws.ptr
            bl.append(b)
        ms = time_fn(va, lambda c, st: va.decode_gqa(fmt, bl[c], Hq, Hkv, L, D, S=S, G=G, stream=st),
                     w.copies, steps, warmup, stream)
        return {"ms": ms, "S": S, "copies": w.copies, "bytes": w.copy_bytes}
    finally:
        w.free()


def bench_paged(va, fmt, B, Hq, Hkv, L, P, D, G, steps, warmup, stream, min_set) -> dict:
    """Paged batch decode (va_decode_paged): B sequences of L positions in pages of
    P rows, pages of a sequence scattered over the pool by a shuffled block table."""
    import numpy as np
    npg = L // P
    num_pages = B * npg
    pay = va.page_bytes(fmt, Hkv, P, D) * num_pages
    sc = va.page_scale_bytes(fmt, Hkv, P, D, G) * num_pages
    per = 2 * (pay + sc)
    copies = max(1, min(256, math.ceil(min_set / per)))
    al = lambda x: (x + 4095) // 4096 * 4096
    pa, sa = al(pay), al(max(sc, 1))
    bufs = []
    def alloc(n):
        bufs.append(va.DeviceBuffer(n))
        return bufs[-1]
    try:
        k, v = alloc(pa * copies), alloc(pa * copies)
        sk = sv = None
        if sc:
            sk, sv = alloc(sa * copies), alloc(sa * copies)
        # copy 0: quantize N(0,1) rows page by page (the layout is the pool's; values only
        # need to be finite), then replicate
        rows = num_pages * Hkv * P
        x = alloc(rows * D * 4)
        bits = va.fmt_bits(fmt)
        for dst, sdst, s in ((k, sk, 11), (v, sv, 12)):
            va.fill_normal(x.ptr, rows * D, s)
            if bits == 16:
                va.f32_to_f16(x.ptr, rows * D, dst.ptr)
            else:
                va.quantize(bits, G, x.ptr, rows, D, dst.ptr, sdst.ptr)
        va.sync()
        for c in range(1, copies):
            for t in (k, v):
                va.check(va.lib.va_memcpy_d2d(t.ptr + c * pa, t.ptr, pay, None))
            if sc:
                for t in (sk, sv):
                    va.check(va.lib.va_memcpy_d2d(t.ptr + c * sa, t.ptr, sc, None))
        table = np.random.default_rng(5).permutation(num_pages).astype(np.int32).reshape(B, npg)
        tab = alloc(table.nbytes)
        tab.upload(table)
        lens = alloc(B * 4)
        lens.upload(np.full(B, L, np.int32))
        q, out = alloc(B * Hq * D * 2), alloc(B * Hq * D * 2)
        va.fill_normal(x.ptr, B * Hq * D, 0x7777)
        va.f32_to_f16(x.ptr, B * Hq * D, q.ptr)
        shape = va.PagedShape(B, Hq, Hkv, D, G, P, npg, num_pages, L)
        S = va.pick_splits_paged(fmt, shape)
        ws = alloc(va.ws_bytes(B * Hq, D, S))
        va.sync()
        bl = [va.PagedBufs(K=k.ptr + c * pa, V=v.ptr + c * pa, scK=sk.ptr + c * sa if sk else 0,
                           scV=sv.ptr + c * sa if sv else 0, block_table=tab.ptr, seq_lens=lens.ptr,
                           q=q.ptr, out=out.ptr, ws=ws.ptr) for c in range(copies)]
        ms = time_fn(va, lambda c, st: va.decode_paged(fmt, bl[c], shape, S, stream=st),
                     copies, steps, warmup, stream)
        return {"ms": ms, "S": S, "copies": copies, "bytes": per}
    finally:
        for b in bufs:
            b.free()


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_reference(H, L, D, G, seconds=2.0) -> dict:
    """The oracle's double-precision reference() (src/voltattn.cu:769-794) on one
    full decode step of q8 inputs (dequantized K/V, format-independent work:
    2*H*L*D MACs), timed on this host: repeated for about `seconds` per line,
    single thread and heads split over T threads; mean and best."""
    import numpy as np
    import oracle
    t0 = time.time()
    c = oracle.make_case(8, H, L, D, G, 0x1234 + L)
    prep_s = time.time() - t0
    kd, vd, q = c["kd"], c["vd"], c["q"]
    threads = max(1, min(H, 16, os.cpu_count() or 1))

    def run(th):
        times, out = [], None
        t_end = time.perf_counter() + seconds
        while not times or time.perf_counter() < t_end:
            t = time.perf_counter()
            out = oracle.reference(kd, vd, q, H, L, D, threads=th)
            times.append(time.perf_counter() - t)
        return out, times

    out1, t1 = run(1)
    outT, tT = run(threads)
    assert np.array_equal(out1, outT)
    mean1, meanT = sum(t1) / len(t1), sum(tT) / len(tT)
    return {
        "ms": mean1 * 1e3, "best_ms": min(t1) * 1e3, "runs": len(t1), "tok_s": 1.0 / mean1,
        "multithread": {"ms": meanT * 1e3, "best_ms": min(tT) * 1e3, "runs": len(tT),
                        "tok_s": 1.0 / meanT, "cores": threads},
        "nproc": os.cpu_count(), "cpu_model": _cpu_model(), "input_prep_s": prep_s,
        "shape": f"q8 H={H} D={D} L={L} G={G}",
    }


def cpu_baseline(H, L, D, G) -> dict:
    """The contract's cpu_baseline: the headline shape on the oracle, 1 core."""
    r = cpu_reference(H, L, D, G, seconds=6.0)
    return {
        "value": r["tok_s"], "unit": "tok/s", "cores": 1, "kind": "port",
        "sample": (f"full decode steps ({r['shape']}): double-precision reference() over the "
                   f"dequantized K/V, {r['runs']} single-thread runs (~6 s), mean"),
        "ms": r["ms"], "best_ms": r["best_ms"],
        "multithread": {"value": r["multithread"]["tok_s"], "unit": "tok/s",
                        "cores": r["multithread"]["cores"], "ms": r["multithread"]["ms"]},
        "nproc": r["nproc"], "cpu_model": r["cpu_model"], "input_prep_s": r["input_prep_s"],
    }


def load_traffic(name: str):
    """HBM bytes per decode launch measured by rocprofv3 FETCH_SIZE + WRITE_SIZE
    (calibrated against a copy of known size), committed in profiles/traffic.json
    by the profiling runs that profiles/*_hbm_traffic.md documents; None if absent."""
    p = ROOT / "profiles" / "traffic.json"
    try:
        entry = json.loads(p.read_text()).get(name)
    except (ValueError, OSError):
        return None
    return None if entry is None else float(entry["traffic_bytes"])


# (config index, format, L); H=32, D=128, G=32.
CONFIG_ROWS = [
    (0, "q8", 4096), (0, "q8+", 4096),
    (1, "f16", 16384), (1, "f16+", 16384),
    (2, "q8+", 16384), (2, "q8+", 65536),
    (3, "q4+", 4096), (3, "q4+", 16384), (3, "q4+", 65536),
    (4, "q3+", 65536), (4, "q3+", 262144),
    (None, "q3+", 16384),                       # q3+ at the metric's shape (not a BASELINE config)
]


def main() -> int:
    global SETTLE_MS
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    # 100 steps keep the timed region of the longest row under 20 ms while the
    # mean stops moving with the launch count (20 steps read 0.5-1 us higher on
    # the 16K rows than 40-100 back to back).
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--G", type=int, default=32)
    ap.add_argument("--H", type=int, default=32)
    ap.add_argument("--D", type=int, default=128)
    ap.add_argument("--headline", default="q8+")
    ap.add_argument("--L", type=int, default=16384, help="the headline's L")
    ap.add_argument("--rows", default="all",
                    help="'all' (every BASELINE config) or a comma list of fmt:L, e.g. q8+:16384,f16+:16384")
    ap.add_argument("--splits", type=int, default=0, help="force S (0: va_pick_splits)")
    ap.add_argument("--warm-ms", type=float, default=50.0,
                    help="untimed steps for at least this long before each row's timed region")
    ap.add_argument("--settle-ms", type=float, default=SETTLE_MS,
                    help="wait after a row's buffers are created, before its first step")
    ap.add_argument("--probe-gib", type=float, default=4.0)
    ap.add_argument("--set-gib", type=float, default=2.0, help="rotated working set per row")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-check", action="store_true", help="skip the after-timing output check")
    ap.add_argument("--steps-only", action="store_true",
                    help="time only the back-to-back steps (no best-single or split-pass launches), so a "
                         "profiler's per-kernel statistics cover fused steps of one shape")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the grouped-query and paged workloads (reported under 'extra')")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="first run one plain device-to-device copy of this many MiB "
                         "(calibrates rocprof FETCH_SIZE/WRITE_SIZE against known bytes)")
    args = ap.parse_args()
    SETTLE_MS = args.settle_ms

    if args.gpus != 1:
        log(f"bench.py: --gpus {args.gpus} is not supported: this build measures one MI355X "
            f"(the decode step would shard by heads or by L across GPUs); run with --gpus 1")
        return 2
    if args.steps < 1:
        log("bench.py: --steps must be >= 1")
        return 2

    import voltattn_amd as va
    info = va.device_info()
    log(f"device: {info['name']} {info['arch']} CUs={info['compute_units']} "
        f"mem={info['total_mem'] / 2**30:.0f} GiB; library {va.LIB_PATH}")
    ceiling = va.probe_read(int(args.probe_gib * 2**30), reps=5)
    log(f"probed read ceiling: {ceiling:.1f} GB/s ({args.probe_gib:g} GiB buffer)")
    launch_floor = va.probe_launch(2000)
    log(f"launch floor: {launch_floor:.2f} us per back-to-back launch of an empty kernel on the decode grid")

    if args.copy_probe_mib > 0:
        nb = args.copy_probe_mib << 20
        src, dst = va.DeviceBuffer(nb), va.DeviceBuffer(nb)
        try:
            va.fill_normal(src.ptr, nb // 4, 7)
            va.sync()
            va.check(va.lib.va_memcpy_d2d(dst.ptr, src.ptr, nb, None))
            va.sync()
        finally:
            src.free()
            dst.free()
        log(f"copy probe: {nb} bytes device-to-device")

    H, D, G = args.H, args.D, args.G
    if args.rows == "all":
        rows_spec = list(CONFIG_ROWS)
    else:
        rows_spec = [(None, x.split(":")[0], int(x.split(":")[1])) for x in args.rows.split(",") if x]
    if not any(f == args.headline and L == args.L for _, f, L in rows_spec):
        rows_spec.append((None, args.headline, args.L))
    stream = va.Stream()
    rows = []
    sized = {}     # algorithmic bytes -> size-matched read ceiling (us, GB/s)
    for cfg, name, L in rows_spec:
        fmt = va.Fmt.parse(name)
        w = Workload(va, fmt, H, L, D, G, int(args.set_gib * 2**30), 256)
        try:
            S = args.splits or va.pick_splits(fmt, H, L, D)
            w.set_splits(S)
            t = time_workload(va, w, args.steps, args.warmup, stream, args.steps_only, args.warm_ms)
            chk = {"checked": None} if args.no_check else check_workload(va, w, (0, H // 2, H - 1))
        finally:
            w.free()
        nbytes = algo_bytes(fmt, H, L, D, G)
        gbs = nbytes / (t["mean_ms"] * 1e6)
        if nbytes not in sized:
            settle()                 # the row's buffers were just freed
            sized[nbytes] = va.probe_read_sized(nbytes, int(args.set_gib * 2**30), launches=max(20, args.steps))
        sz_us, sz_gbs = sized[nbytes]
        r = {"config": cfg, "fmt": fmt.label, "L": L, "S": S,
             "ms": t["mean_ms"], "best_single_ms": t["best_ms"], "split_pass_ms": t["kernel_ms"],
             "tok_s": 1e3 / t["mean_ms"], "tok_s_best_single": 1e3 / t["best_ms"],
             "bytes": nbytes, "gbps": gbs, "mbu": gbs / ceiling, "pct_peak": gbs / PEAK_HBM_GBPS,
             "sized_ceiling_us": sz_us, "sized_ceiling_gbps": sz_gbs, "mbu_sized": gbs / sz_gbs,
             "copies": w.copies, "working_set_bytes": w.copies * w.copy_bytes, **chk}
        rows.append(r)
        log(f"cfg[{'-' if cfg is None else cfg}] {fmt.label:5s} L={L:6d} S={S:3d} copies={w.copies:3d}  "
            f"mean {r['ms'] * 1e3:8.2f} us  best {r['best_single_ms'] * 1e3:8.2f} us  "
            f"{gbs:7.1f} GB/s  MBU {100 * r['mbu']:5.1f}%  peak {100 * r['pct_peak']:5.1f}%  "
            f"sized read {sz_us:7.2f} us ({100 * r['mbu_sized']:5.1f}%)  "
            f"tok/s {r['tok_s']:8.0f}  check {'-' if r['checked'] is None else ('ok' if r['checked'] else 'FAIL')}")
    # vs f16 / vs f16+ at the same L
    for r in rows:
        for ref_fmt, key in (("f16", "vs_f16"), ("f16+", "vs_f16p")):
            base = [x for x in rows if x["fmt"] == ref_fmt and x["L"] == r["L"]]
            if base:
                r[key] = base[0]["ms"] / r["ms"]
    formats = {r["fmt"]: r for r in rows if r["L"] == args.L}

    extra = {}
    if not args.no_extra:
        # Beyond the reference (grouped-query attention, paged batches): same bytes
        # definition (K+V payload + scales actually read), tok/s per decode step.
        min_set = int(args.set_gib * 2**30)
        specs = [("gqa", "q8+", dict(Hq=32, Hkv=8, L=65536)), ("gqa", "f16+", dict(Hq=32, Hkv=8, L=65536)),
                 ("gqa", "q4+", dict(Hq=32, Hkv=8, L=65536)), ("gqa", "q3+", dict(Hq=32, Hkv=8, L=65536)),
                 ("paged", "q8+", dict(B=8, Hq=32, Hkv=8, L=16384, P=256)),
                 ("paged", "q4+", dict(B=8, Hq=32, Hkv=8, L=16384, P=256)),
                 ("paged", "q3+", dict(B=8, Hq=32, Hkv=8, L=16384, P=256)),
                 ("paged", "q8+", dict(B=1, Hq=32, Hkv=32, L=16384, P=256)),
                 ("paged", "f16+", dict(B=1, Hq=32, Hkv=32, L=16384, P=256))]
        for kind, name, p in specs:
            fmt = va.Fmt.parse(name)
            if kind == "gqa":
                r = bench_gqa(va, fmt, p["Hq"], p["Hkv"], p["L"], D, G, args.steps, args.warmup, stream, min_set)
                key = f"gqa {name} Hq={p['Hq']} Hkv={p['Hkv']} L={p['L']}"
                seqs = 1
            else:
                r = bench_paged(va, fmt, p["B"], p["Hq"], p["Hkv"], p["L"], p["P"], D, G, args.steps,
                                args.warmup, stream, min_set)
                key = f"paged {name} B={p['B']} Hq={p['Hq']} Hkv={p['Hkv']} L={p['L']} page={p['P']}"
                seqs = p["B"]
            gbs = r["bytes"] / (r["ms"] * 1e6)
            extra[key] = {"ms": r["ms"], "tok_s": seqs * 1e3 / r["ms"], "gbps": gbs, "mbu": gbs / ceiling,
                          "bytes": r["bytes"], "S": r["S"], "copies": r["copies"]}
            log(f"{key:48s} S={r['S']:3d}  mean {r['ms'] * 1e3:8.2f} us  {gbs:7.1f} GB/s  "
                f"MBU {100 * gbs / ceiling:5.1f}%  tok/s {seqs * 1e3 / r['ms']:8.0f}")
    stream.destroy()

    head = formats[args.headline]
    # The step is one launch of the fused kernel (split-L pass + last-group LSE
    # merge), so its mean back-to-back duration over the timed region is the
    # kernel's launch duration; the split pass alone is reported beside it.
    step_gbs = head["gbps"]
    roofline = {"bound": "hbm", "achieved": step_gbs, "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                "frac": step_gbs / PEAK_HBM_GBPS, "traffic": load_traffic(f"{args.headline}_L{args.L}_G{G}"),
                "kernel": f"{HEADLINE_KERNEL.get(args.headline, 'decode_tiled')}<{args.headline}> fused "
                          "(split-L pass + LSE merge, one launch per step)",
                "algorithmic_bytes_per_launch": head["bytes"],
                "kernel_ms": head["ms"], "frac_of_probed": step_gbs / ceiling,
                "frac_of_sized_read": head["mbu_sized"], "sized_read_us": head["sized_ceiling_us"],
                "split_pass_only_ms": head["split_pass_ms"],
                "split_pass_only_gbps": head["bytes"] / (head["split_pass_ms"] * 1e6) if head["split_pass_ms"] > 0 else None}
    cpu = cpu0 = None
    if not args.no_cpu:
        cpu = cpu_baseline(H, args.L, D, G)
        log(f"cpu baseline ({cpu['cpu_model']}, nproc {cpu['nproc']}): L={args.L}: {cpu['value']:.2f} tok/s "
            f"on 1 core ({cpu['ms']:.1f} ms), {cpu['multithread']['value']:.1f} tok/s on "
            f"{cpu['multithread']['cores']} threads ({cpu['multithread']['ms']:.2f} ms)")
        cpu0 = cpu_reference(H, 4096, D, G, seconds=3.0)
        g0 = {r["fmt"]: r for r in rows if r["L"] == 4096}
        cpu0["gpu_rows"] = {f: {"ms": g0[f]["ms"], "tok_s": g0[f]["tok_s"]} for f in ("q8", "q8+") if f in g0}
        log(f"configs[0] CPU path (q8 L=4096): {cpu0['ms']:.2f} ms = {cpu0['tok_s']:.1f} tok/s on 1 core, "
            f"{cpu0['multithread']['ms']:.2f} ms = {cpu0['multithread']['tok_s']:.1f} tok/s on "
            f"{cpu0['multithread']['cores']} threads; GPU " +
            ", ".join(f"{f} {v['ms'] * 1e3:.1f} us = {v['tok_s']:.0f} tok/s" for f, v in cpu0["gpu_rows"].items()))

    checked = None if args.no_check else all(r["checked"] for r in rows)
    line = {
        "metric": METRIC, "value": head["tok_s"], "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": head["ms"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32", "data": "synthetic",
        "config": {"workload": f"{args.headline} decode step, batch 1, H={H} D={D} L={args.L} G={G} "
                               f"(BASELINE configs[2] shape; the metric's H32 D128 L16K)",
                   "H": H, "D": D, "L": args.L, "G": G, "S": head["S"], "copies": head["copies"],
                   "storage": {"f16": "fp16", "f16+": "fp16", "q8": "int8", "q8+": "int8",
                               "q4": "int4", "q4+": "int4", "q3+": "int3"}[args.headline],
                   "parallelism": "single GPU, split-L"},
        "checked": checked,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "cpu_configs0": cpu0,
        "probed_ceiling_gbps": ceiling,
        "launch_floor_us": launch_floor,
        "mbu": head["mbu"],
        "formats": formats,
        "configs": rows,
        "extra": extra,
        "device": info["name"] or info["arch"], "arch": info["arch"], "compute_units": info["compute_units"],
    }
    print(json.dumps(line), flush=True)
    if checked is False:
        log("bench.py: an output check FAILED: " +
            ", ".join(f"{r['fmt']} L={r['L']}" for r in rows if not r["checked"]))
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
