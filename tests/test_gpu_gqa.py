"""GPU parity of grouped-query decode (va_decode_gqa) through the C ABI.

Query head h attends KV head h // (Hq/Hkv); the expected output is the
oracle's double reference over the repeated KV heads (oracle.batch, pinned in
test_oracle_batch.py). Gates per output: the reference's rule
|got - ref| <= 3e-3 + 2e-2|ref| (src/voltattn.cu:903) and the tight bound
(half an fp16 ulp + 2e-6|ref|, tests/numerics.py). Group sizes cover powers of
two, odd groups (masked query slots) and groups larger than a work-group's
slots (several sub-groups per KV head)."""
import numpy as np
import pytest

import oracle
from oracle import batch
import voltattn_amd as va
from tests import batch_util
from tests.numerics import tight_bound

pytestmark = pytest.mark.gpu

TILED = [va.Fmt.F16M, va.Fmt.Q8M, va.Fmt.Q4M, va.Fmt.Q3M]
HEADS = [(8, 2), (8, 1), (12, 4), (14, 2), (16, 2), (6, 3)]


def _run(fmt, Hq, Hkv, L, D, G, S, seed):
    c = batch_util.kv_case(fmt, Hkv, L, D, G, seed)
    q = batch_util.queries(Hq, D, seed + 5)
    bufs = []
    try:
        dev = lambda a: bufs.append(va.DeviceBuffer.from_array(a)) or bufs[-1].ptr
        Sx = S or va.pick_splits_gqa(fmt, Hq, Hkv, L, D)
        out = va.DeviceBuffer(Hq * D * 2)
        ws = va.DeviceBuffer(va.ws_bytes(Hq, D, max(Sx, 1)))
        bufs += [out, ws]
        b = va.DeviceBufs(K=dev(c["kpay"]), V=dev(c["vpay"]),
                          scK=dev(c["ksc"]) if c["ksc"] is not None else 0,
                          scV=dev(c["vsc"]) if c["vsc"] is not None else 0,
                          q=dev(q), out=out.ptr, ws=ws.ptr)
        va.decode_gqa(fmt, b, Hq, Hkv, L, D, S=S, G=G)
        va.sync()
        got = out.download(np.uint16).view(np.float16).astype(np.float32)
    finally:
        for x in bufs:
            x.free()
    ref = batch.reference_gqa(c["kd"], c["vd"], q, Hq, Hkv, L, D)
    return got, ref


def _check(got, ref, what):
    assert np.all(np.isfinite(got)), what
    ok, maxerr = oracle.gate(got, ref)
    assert ok, (what, maxerr)
    bad = np.abs(got - ref) > tight_bound(ref)
    assert not bad.any(), (what, int(bad.sum()), float(np.abs(got - ref).max()))


@pytest.mark.parametrize("fmt", TILED, ids=lambda f: f.label)
@pytest.mark.parametrize("heads", HEADS, ids=lambda h: f"Hq{h[0]}-Hkv{h[1]}")
@pytest.mark.parametrize("L", [257, 3000])
def test_gqa_matches_oracle(fmt, heads, L):
    Hq, Hkv = heads
    print(f"gqa {fmt.label} Hq={Hq} Hkv={Hkv} L={L}", flush=True)
    got, ref = _run(fmt, Hq, Hkv, L, 128, 32, 0, 0x6A0 + Hq * 31 + L)
    _check(got, ref, (fmt.label, Hq, Hkv, L))


@pytest.mark.parametrize("fmt", TILED, ids=lambda f: f.label)
@pytest.mark.parametrize("S", [1, 3, 64, 100])      # 100 > 64: two-pass form (merge kernel)
def test_gqa_split_counts(fmt, S):
    print(f"gqa splits {fmt.label} S={S}", flush=True)
    got, ref = _run(fmt, 8, 2, 2049, 128, 32, S, 0x51 + S)
    _check(got, ref, (fmt.label, S))


@pytest.mark.parametrize("fmt", TILED, ids=lambda f: f.label)
def test_gqa_d64_g64(fmt):
    print(f"gqa d64 {fmt.label}", flush=True)
    got, ref = _run(fmt, 8, 2, 513, 64, 64, 0, 0x64)
    _check(got, ref, fmt.label)


@pytest.mark.parametrize("fmt", TILED, ids=lambda f: f.label)
def test_gqa_d128_g64(fmt):
    # two scale groups per row: the matrix-core forms stack NG = 2 columns per query slot
    print(f"gqa d128 g64 {fmt.label}", flush=True)
    got, ref = _run(fmt, 12, 3, 1500, 128, 64, 0, 0x12864)
    _check(got, ref, fmt.label)


@pytest.mark.parametrize("fmt", TILED, ids=lambda f: f.label)
def test_paged_d128_g64(fmt):
    print(f"paged d128 g64 {fmt.label}", flush=True)
    pb = batch_util.PagedBatch(fmt, [700, 1, 1300], 8, 2, 128, 64, 256, seed=0x6464)
    try:
        got = pb.run()
    finally:
        pb.free()
    for b in range(3):
        _check(got[b].astype(np.float32).ravel(), pb.ref[b].ravel(), (fmt.label, "paged", b))


def test_gqa_single_position():
    got, ref = _run(va.Fmt.Q8M, 8, 2, 1, 128, 32, 0, 0x1)
    _check(got, ref, "L=1")


def test_gqa_equal_heads_is_va_decode():
    """Hq == Hkv routes to va_decode: bit-identical outputs."""
    fmt, H, L, D, G = va.Fmt.Q8M, 4, 700, 128, 32
    c = batch_util.kv_case(fmt, H, L, D, G, 0x77)
    q = batch_util.queries(H, D, 0x78)
    S = va.pick_splits(fmt, H, L, D)
    outs = []
    for use_gqa in (False, True):
        bufs = [va.DeviceBuffer.from_array(a) for a in (c["kpay"], c["vpay"], c["ksc"], c["vsc"], q)]
        out, ws = va.DeviceBuffer(H * D * 2), va.DeviceBuffer(va.ws_bytes(H, D, S))
        try:
            b = va.DeviceBufs(K=bufs[0].ptr, V=bufs[1].ptr, scK=bufs[2].ptr, scV=bufs[3].ptr,
                              q=bufs[4].ptr, out=out.ptr, ws=ws.ptr)
            if use_gqa:
                va.decode_gqa(fmt, b, H, H, L, D, S=S, G=G)
            else:
                va.launch(fmt, b, H, L, D, S, G=G)
            va.sync()
            outs.append(out.download(np.uint16))
        finally:
            for x in bufs + [out, ws]:
                x.free()
    np.testing.assert_array_equal(outs[0], outs[1])


# Grouped f16+ runs the two-phase kernel (va_phased.hpp), whose rounds hold
# 8192 / QG positions: splits of several rounds with a ragged last one, at four
# query slots (Hq 8 / Hkv 2), two (Hq 4 / Hkv 2) and a group of three with one
# masked slot (Hq 6 / Hkv 2).
@pytest.mark.parametrize("shape", [(8, 2, 20000, 2), (4, 2, 9000, 1), (6, 2, 7000, 1)],
                         ids=lambda s: "Hq{}-Hkv{}-L{}-S{}".format(*s))
def test_gqa_f16_multi_round(shape):
    Hq, Hkv, L, S = shape
    print(f"gqa f16+ rounds Hq={Hq} Hkv={Hkv} L={L} S={S}", flush=True)
    got, ref = _run(va.Fmt.F16M, Hq, Hkv, L, 128, 32, S, 0x7A0 + L)
    _check(got, ref, ("f16+ rounds", Hq, Hkv, L, S))
