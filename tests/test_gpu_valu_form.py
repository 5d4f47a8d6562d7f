"""GPU: the vector-ALU form of grouped and paged q8+/q4+ decode, and of q3+ at D = 128.

The product runs these on the matrix cores; the vector-ALU kernels are built
into a comparison library (build/variants/libvoltattn_hip_valu.so, compiled
with VA_GQA_MFMA=0), so the cases run in one child process that loads it
(tests/variant_pkg.py): grouped-query decode (four query slots per work-group
for q8+, two for q4+ and q3+, sub-groups and masked slots) at D = 128 and 64
(q3+: D = 128, the only width it runs on the matrix cores in the product) and
G = 32 and 64, and paged batches with ragged lengths, each against the
oracle's double reference (oracle.batch) within the reference's gate
(src/voltattn.cu:903) and the fp16 rounding bound. The matrix-core form of the
same cases is covered by test_gpu_gqa.py and test_gpu_paged.py."""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
pytestmark = pytest.mark.gpu
N_CASES = 36


def _child() -> None:
    import numpy as np

    import oracle
    from oracle import batch
    import voltattn_amd as va
    from tests import batch_util
    from tests.numerics import tight_bound

    def check(got, ref, what):
        assert np.all(np.isfinite(got)), what
        ok, maxerr = oracle.gate(got.ravel(), ref.ravel())
        assert ok, (what, maxerr)
        bad = np.abs(got - ref) > tight_bound(ref)
        assert not bad.any(), (what, int(bad.sum()), float(np.abs(got - ref).max()))

    assert "va_valu_" in str(va.LIB_PATH), va.LIB_PATH      # the comparison build, not the product
    n = 0
    shapes = [(Hq, Hkv, L, 128, 32) for Hq, Hkv in ((8, 2), (12, 4), (16, 2), (6, 3)) for L in (257, 3000)]
    # other scale layouts: one scale group per lane row (D = 64, G = 64), two (D = 128, G = 64)
    shapes += [(8, 2, 3000, 64, 32), (12, 4, 1000, 64, 64), (8, 2, 2000, 128, 64), (6, 3, 777, 64, 32)]
    for fmt in (va.Fmt.Q8M, va.Fmt.Q4M, va.Fmt.Q3M):
        for Hq, Hkv, L, D, G in shapes:
            if fmt == va.Fmt.Q3M and D != 128:
                continue
            print(f"valu gqa {fmt.label} Hq={Hq} Hkv={Hkv} L={L} D={D} G={G}", flush=True)
            seed = 0x7A1 + Hq * 31 + L
            c = batch_util.kv_case(fmt, Hkv, L, D, G, seed)
            q = batch_util.queries(Hq, D, seed + 5)
            bufs = []
            try:
                dev = lambda a: bufs.append(va.DeviceBuffer.from_array(a)) or bufs[-1].ptr
                S = va.pick_splits_gqa(fmt, Hq, Hkv, L, D)
                out = va.DeviceBuffer(Hq * D * 2)
                ws = va.DeviceBuffer(va.ws_bytes(Hq, D, S))
                bufs += [out, ws]
                b = va.DeviceBufs(K=dev(c["kpay"]), V=dev(c["vpay"]), scK=dev(c["ksc"]),
                                  scV=dev(c["vsc"]), q=dev(q), out=out.ptr, ws=ws.ptr)
                va.decode_gqa(fmt, b, Hq, Hkv, L, D, S=0, G=G)
                va.sync()
                got = out.download(np.uint16).view(np.float16).astype(np.float64)
            finally:
                for x in bufs:
                    x.free()
            ref = batch.reference_gqa(c["kd"], c["vd"], q, Hq, Hkv, L, D).astype(np.float64)
            check(got.reshape(ref.shape), ref, (fmt.label, Hq, Hkv, L, D, G))
            n += 1
        lens = [1, 63, 65, 300, 1500]
        print(f"valu paged {fmt.label} lens={lens}", flush=True)
        pb = batch_util.PagedBatch(fmt, lens, 8, 2, 128, 32, 64, seed=0x7B)
        try:
            got = pb.run()
        finally:
            pb.free()
        for b in range(len(lens)):
            check(got[b].astype(np.float64).ravel(), pb.ref[b].astype(np.float64).ravel(),
                  (fmt.label, "paged", b))
        n += 1
    print(f"valu form: {n} cases passed", flush=True)


def test_valu_form_grouped_and_paged():
    from tests.variant_pkg import run_child
    r = run_child("valu", Path(__file__).resolve())
    print(r.stdout[-2000:], r.stderr[-2000:])
    assert r.returncode == 0, r.stderr[-2000:]
    assert f"valu form: {N_CASES} cases passed" in r.stdout


if __name__ == "__main__" and "--child" in sys.argv:
    _child()
