"""GPU: the failure path of the fused merge, forced by a test build.

A comparison library (build/variants/libvoltattn_hip_lost.so, both kernel
units compiled with VA_TEST_LOSE_MERGES=1) makes every fused merge wait for
something that never comes: a tag no partial carries (one query slot, the
tagged protocol) or one more count than there are groups (several slots, the
counted protocol). Each merge therefore gives up after its bounded wait; every
kernel still exits normally. Checked in one child process (tests/variant_pkg.py):

* the outputs of those merges are NaN (fp16 0x7E00) and nothing else;
* va_merge_faults returns VA_ELOST with exactly one loss per merge group, and
  the next call returns VA_OK with 0 (each loss is reported once);
* the ticket slot is left consistent: the same stream's next calls give up the
  same way (no stale count or tag carries over);
* the two-pass form (S > 64: partials in ws, separate merge kernel) has no
  in-kernel merge, so it stays within the fp16 rounding bound of the oracle's
  double reference and reports no loss."""
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu
VA_OK, VA_ELOST = 0, 7


def _child() -> None:
    import ctypes as C

    import numpy as np

    import voltattn_amd as va
    from tests import batch_util, gpu_util
    from tests.numerics import tight_bound

    assert "va_lost_" in str(va.LIB_PATH), va.LIB_PATH      # the test build, not the product
    st = va.Stream()

    def faults():
        n = C.c_uint(0)
        rc = va.lib.va_merge_faults(C.c_void_p(st.handle), C.byref(n))
        return rc, n.value

    def decode(fmt, c, S):
        H, L, D, G = c["H"], c["L"], c["D"], c["G"]
        bufs = []
        try:
            dev = lambda a: bufs.append(va.DeviceBuffer.from_array(a)) or bufs[-1].ptr
            out = va.DeviceBuffer(H * D * 2)
            ws = va.DeviceBuffer(va.ws_bytes(H, D, S))
            bufs += [out, ws]
            b = va.DeviceBufs(K=dev(c["kpay"]), V=dev(c["vpay"]),
                              scK=dev(c["ksc"]) if c["ksc"] is not None else 0,
                              scV=dev(c["vsc"]) if c["vsc"] is not None else 0,
                              q=dev(c["q"]), out=out.ptr, ws=ws.ptr)
            va.launch(fmt, b, H, L, D, S, G=G, stream=st)
            st.synchronize()
            return out.download(np.uint16)
        finally:
            for x in bufs:
                x.free()

    assert faults() == (VA_OK, 0)
    # one query slot (tagged protocol): 4- and 8-wave groups, one merge per head
    for fmt, H, L, S in ((va.Fmt.Q8M, 6, 3000, 5), (va.Fmt.F16M, 4, 2000, 3), (va.Fmt.Q3M, 3, 2500, 7)):
        c = gpu_util.case(va.fmt_bits(fmt), H, L, 128, 32, 0x10CE + H)
        for rep in range(2):                     # the slot is consistent for the next call
            print(f"lost merge: {fmt.label} H={H} L={L} S={S} call {rep}", flush=True)
            got = decode(fmt, c, S)
            assert np.all(got == 0x7E00), (fmt.label, rep)
            assert faults() == (VA_ELOST, H), (fmt.label, rep)
            assert faults() == (VA_OK, 0)
    # several query slots (counted protocol): Hq 8 over Hkv 2, one merge per KV head
    for fmt in (va.Fmt.Q8M, va.Fmt.F16M):
        Hq, Hkv, L, D, G = 8, 2, 3000, 128, 32
        print(f"lost merge: grouped {fmt.label} Hq={Hq} Hkv={Hkv} L={L}", flush=True)
        kv = batch_util.kv_case(fmt, Hkv, L, D, G, 0x10CF)
        q = batch_util.queries(Hq, D, 0x10D0)
        bufs = []
        try:
            dev = lambda a: bufs.append(va.DeviceBuffer.from_array(a)) or bufs[-1].ptr
            S = va.pick_splits_gqa(fmt, Hq, Hkv, L, D)
            out = va.DeviceBuffer(Hq * D * 2)
            ws = va.DeviceBuffer(va.ws_bytes(Hq, D, S))
            bufs += [out, ws]
            b = va.DeviceBufs(K=dev(kv["kpay"]), V=dev(kv["vpay"]),
                              scK=dev(kv["ksc"]) if kv["ksc"] is not None else 0,
                              scV=dev(kv["vsc"]) if kv["vsc"] is not None else 0,
                              q=dev(q), out=out.ptr, ws=ws.ptr)
            va.decode_gqa(fmt, b, Hq, Hkv, L, D, S=S, G=G, stream=st)
            st.synchronize()
            got = out.download(np.uint16)
        finally:
            for x in bufs:
                x.free()
        assert S <= 64, S                        # the fused form
        assert np.all(got == 0x7E00), fmt.label
        assert faults() == (VA_ELOST, Hkv), fmt.label    # one per KV head (4 query heads: one sub-group)
        assert faults() == (VA_OK, 0)
    # two-pass form: no in-kernel merge, nothing to lose
    fmt, H, L, S = va.Fmt.Q8M, 4, 3000, 80
    print(f"two-pass: {fmt.label} H={H} L={L} S={S}", flush=True)
    c = gpu_util.case(va.fmt_bits(fmt), H, L, 128, 32, 0x10D1)
    got = decode(fmt, c, S).view(np.float16).astype(np.float64)
    ref = c["ref"].astype(np.float64)
    assert np.all(np.abs(got - ref) <= tight_bound(ref))
    assert faults() == (VA_OK, 0)
    st.destroy()
    print("lost merges: ok", flush=True)


def test_lost_merges_are_nan_and_counted_once():
    from tests import variant_pkg
    r = variant_pkg.run_child("lost", Path(__file__))
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    assert "lost merges: ok" in r.stdout, r.stdout[-3000:]


if __name__ == "__main__" and "--child" in sys.argv:
    _child()
