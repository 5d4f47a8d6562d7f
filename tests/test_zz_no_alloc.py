"""GPU: va_decode_noalloc, the allocation-free form of va_decode.

It takes no workspace: the two-pass form's partials go to a file-scope device
array of the library (VA_NOALLOC_MAX_FLOATS floats per device) whose address
is looked up once per device. Through the C ABI, its outputs must equal
va_decode's (same kernels, caller-provided ws) bit for bit, on consecutive
calls with the second smaller than the first, both in the fused form (merge
inside the decode kernel; the workspace is unused) and in the two-pass form
(S > 64: partials through the library workspace, then the merge kernel), and
inside the reference's gate against the oracle. Shapes whose partials exceed
the workspace are refused with VA_ERANGE before any device work.

The workspace has one owner at a time (tests/noalloc_child.py, in a fresh
process so that every ticket slot can be bound by captured graphs and the
two-pass form is forced at S <= 64): another stream's call is refused with
VA_EBUSY while the owner's work may still run, the binding moves once the
owner is idle (eager streams) or released (per-thread streams, captures), and
every output stays exact."""
import ctypes as C
import os
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

import oracle
import voltattn_amd as va
from tests import gpu_util

pytestmark = pytest.mark.gpu

MAX_FLOATS = 1048576          # VA_NOALLOC_MAX_FLOATS (include/voltattn.h)


def _run(fmt, c, S, noalloc):
    H, L, D, G = c["H"], c["L"], c["D"], c["G"]
    bufs = []
    try:
        dev = lambda a: bufs.append(va.DeviceBuffer.from_array(a)) or bufs[-1].ptr
        out = va.DeviceBuffer(H * D * 2)
        bufs.append(out)
        ws = 0
        if not noalloc:
            w = va.DeviceBuffer(va.ws_bytes(H, D, S))
            bufs.append(w)
            ws = w.ptr
        b = va.DeviceBufs(K=dev(c["kpay"]), V=dev(c["vpay"]),
                          scK=dev(c["ksc"]) if c["ksc"] is not None else 0,
                          scV=dev(c["vsc"]) if c["vsc"] is not None else 0,
                          q=dev(c["q"]), out=out.ptr, ws=ws)
        cb = b._c()
        fn = va.lib.va_decode_noalloc if noalloc else va.lib.va_decode
        va.check(fn(int(fmt), C.byref(cb), H, L, D, G, S, None))
        va.sync()
        return out.download(np.uint16)
    finally:
        for x in bufs:
            x.free()


# (H, L, S): the second call of each pair is smaller; S > 64 takes the two-pass form
PAIRS = {"fused": [(16, 5000, 8), (4, 1200, 3)], "two_pass": [(16, 5000, 80), (4, 1200, 70)]}


@pytest.mark.parametrize("form", sorted(PAIRS))
@pytest.mark.parametrize("fmt", [va.Fmt.Q8M, va.Fmt.F16M, va.Fmt.Q4M, va.Fmt.Q3M, va.Fmt.Q8],
                         ids=lambda f: f.label)
def test_noalloc_matches_decode(fmt, form):
    for i, (H, L, S) in enumerate(PAIRS[form]):
        assert H * S * (128 + 2) <= MAX_FLOATS
        print(f"noalloc {fmt.label} {form} call {i}: H={H} L={L} S={S}", flush=True)
        c = gpu_util.case(va.fmt_bits(fmt), H, L, 128, 32, 0xA110C + 17 * i + H)
        want = _run(fmt, c, S, noalloc=False)
        got = _run(fmt, c, S, noalloc=True)
        assert np.array_equal(got, want), (fmt.label, form, i)
        ok, maxerr = oracle.gate(got.view(np.float16).astype(np.float64), c["ref"])
        assert ok, maxerr


def test_noalloc_refuses_oversized_workspace():
    b = va.DeviceBufs(K=1 << 20, V=1 << 20, scK=1 << 20, scV=1 << 20, q=1 << 20, out=1 << 20)
    cb = b._c()
    H, S, D = 1024, 64, 128                       # 1024*64*130 floats > the workspace
    assert H * S * (D + 2) > MAX_FLOATS
    rc = va.lib.va_decode_noalloc(int(va.Fmt.Q8M), C.byref(cb), H, 4096, D, 32, S, None)
    assert rc == 4, va.lib.va_last_error()        # VA_ERANGE
    assert b"exceeds the allocation-free workspace" in va.lib.va_last_error()


def test_noalloc_workspace_has_one_owner():
    env = dict(os.environ)
    env.pop("VOLTATTN_HIP_RUNTIME", None)          # the child uses no torch
    root = Path(__file__).resolve().parent.parent
    print("noalloc workspace ownership (child process)", flush=True)
    r = subprocess.run([sys.executable, "-u", str(root / "tests" / "noalloc_child.py")], cwd=root, env=env,
                       capture_output=True, text=True, timeout=110)
    print(r.stdout[-3000:], flush=True)
    assert r.returncode == 0, r.stderr[-3000:]
    assert "noalloc child: ok" in r.stdout
