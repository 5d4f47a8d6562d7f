"""GPU parity of paged, batched decode (va_decode_paged) and of the cache write
path (va_append_kv) through the C ABI.

Each sequence's rows are scattered through a shuffled block table into a page
pool whose other rows hold random bytes (fp16 NaN/Inf patterns included), so
a read past a sequence's length or through the wrong page shows up. Expected
outputs: the oracle's double reference over each sequence's dequantized rows
(oracle.batch); gates as in test_gpu_gqa.py. The appended cache must equal,
byte for byte, the oracle's quantizer (quantize(), src/voltattn.cu:705-745)
applied to the same fp16 rows, placed at the table's rows."""
import numpy as np
import pytest

import oracle
from oracle import batch
import voltattn_amd as va
from tests import batch_util
from tests.numerics import tight_bound

pytestmark = pytest.mark.gpu

TILED = [va.Fmt.F16M, va.Fmt.Q8M, va.Fmt.Q4M, va.Fmt.Q3M]


def _check(got, ref, what):
    assert np.all(np.isfinite(got)), what
    ok, maxerr = oracle.gate(got, ref)
    assert ok, (what, maxerr)
    bad = np.abs(got - ref) > tight_bound(ref)
    assert not bad.any(), (what, int(bad.sum()), float(np.abs(got - ref).max()))


@pytest.mark.parametrize("fmt", TILED, ids=lambda f: f.label)
@pytest.mark.parametrize("page_rows", [64, 256])
@pytest.mark.parametrize("heads", [(8, 2), (4, 4), (14, 2)], ids=lambda h: f"Hq{h[0]}-Hkv{h[1]}")
def test_paged_batch_matches_oracle(fmt, page_rows, heads):
    Hq, Hkv = heads
    lens = [1, 63, 64, 65, 300, 1500]
    print(f"paged {fmt.label} P={page_rows} Hq={Hq} Hkv={Hkv} lens={lens}", flush=True)
    pb = batch_util.PagedBatch(fmt, lens, Hq, Hkv, 128, 32, page_rows, seed=page_rows + Hq)
    try:
        got = pb.run()
    finally:
        pb.free()
    for b in range(len(lens)):
        _check(got[b].ravel(), pb.ref[b].ravel(), (fmt.label, b, lens[b]))


@pytest.mark.parametrize("fmt", TILED, ids=lambda f: f.label)
@pytest.mark.parametrize("S", [1, 5, 64, 80])      # 80 > 64: two-pass form
def test_paged_split_counts(fmt, S):
    lens = [2000, 517, 1]
    print(f"paged splits {fmt.label} S={S}", flush=True)
    pb = batch_util.PagedBatch(fmt, lens, 8, 2, 128, 32, 64, seed=S)
    try:
        got = pb.run(S=S)
    finally:
        pb.free()
    for b in range(len(lens)):
        _check(got[b].ravel(), pb.ref[b].ravel(), (fmt.label, S, b))


@pytest.mark.parametrize("fmt", TILED, ids=lambda f: f.label)
@pytest.mark.parametrize("page_rows", [64, 128])
def test_paged_d64_g64(fmt, page_rows):
    """D = 64 at the smallest page: q4 reads 32 rows per wave load, so its wave
    tile must shrink to stay inside one 64-row page."""
    print(f"paged d64 {fmt.label} P={page_rows}", flush=True)
    pb = batch_util.PagedBatch(fmt, [700, 129, 64], 8, 2, 64, 64, page_rows, seed=9 + page_rows)
    try:
        got = pb.run()
    finally:
        pb.free()
    for b in range(3):
        _check(got[b].ravel(), pb.ref[b].ravel(), (fmt.label, b))


def test_paged_many_sequences_two_pass():
    """B*Hq*S beyond the fused merge's partial store: the merge kernel path."""
    lens = list(np.random.default_rng(3).integers(1, 600, 40))
    pb = batch_util.PagedBatch(va.Fmt.Q8M, lens, 32, 8, 128, 32, 64, seed=11)
    try:
        got = pb.run(S=4)           # 40*8 groups x 4 slots x 4 splits = 5120 partials > 2048
    finally:
        pb.free()
    for b in range(len(lens)):
        _check(got[b].ravel(), pb.ref[b].ravel(), b)


# (format, Hq, Hkv, page rows): the grouped-query kernels, and one query slot per
# KV head with pages that hold a whole work-group tile of the two-phase kernel
BAD_INPUT_CASES = [(va.Fmt.Q8M, 8, 2, 64), (va.Fmt.Q8M, 2, 2, 128), (va.Fmt.F16M, 2, 2, 64)]


@pytest.mark.parametrize("case", BAD_INPUT_CASES, ids=lambda c: f"{c[0].label}-Hq{c[1]}-Hkv{c[2]}-P{c[3]}")
@pytest.mark.parametrize("S", [0, 80])              # 0: fused merge; 80 > 64: the merge kernel
def test_paged_empty_bad_page_and_overlong_sequence(S, case):
    """Length 0 -> zeros; a page id outside the pool, a length above
    max_seq_len or a negative length -> NaN for that sequence only; the others
    stay exact. Both merge paths (in the decode kernel and the separate
    lse_merge pass) give the same verdicts."""
    fmt, Hq, Hkv, P = case
    lens = [300, 0, 300, 300, 0]
    pb = batch_util.PagedBatch(fmt, lens, Hq, Hkv, 128, 32, P, seed=5, max_seq_len=320,
                               max_pages=384 // P)
    try:
        table = pb.table.copy()
        table[2, 1] = pb.shape.num_pages + 5          # sequence 2: second page id outside the pool
        seq = pb.seq_lens.copy()
        seq[3] = 321                                  # sequence 3: above max_seq_len
        seq[4] = -5                                   # sequence 4: negative length
        print(f"paged bad inputs S={S} {fmt.label} Hq={Hq} Hkv={Hkv} P={P}", flush=True)
        got = pb.run(S=S, table=table, seq_lens=seq)
    finally:
        pb.free()
    _check(got[0].ravel(), pb.ref[0].ravel(), 0)
    assert np.all(got[1] == 0.0)
    assert np.all(np.isnan(got[2]))
    assert np.all(np.isnan(got[3]))
    assert np.all(np.isnan(got[4]))


def test_contiguous_cache_as_one_page_per_sequence():
    """A contiguous cache [Hkv][Lcap][row] per sequence is page_rows = Lcap with
    block_table[b] = {b}: same result as va_decode_gqa on each sequence."""
    fmt, Hq, Hkv, D, G, Lcap = va.Fmt.Q8M, 8, 2, 128, 32, 1024
    lens = [1024, 700]
    pb = batch_util.PagedBatch(fmt, lens, Hq, Hkv, D, G, Lcap, seed=21, extra_pages=0)
    pb.table = np.arange(2, dtype=np.int32).reshape(2, 1)
    # rebuild the pool in table order so that page b is sequence b's contiguous cache
    for b, L in enumerate(lens):
        c = batch_util.kv_case(fmt, Hkv, L, D, G, 21 * 7919 + b)
        pb.kpool[b, :, :L], pb.vpool[b, :, :L] = c["kpay"], c["vpay"]
        pb.kspool[b, :, :L], pb.vspool[b, :, :L] = c["ksc"], c["vsc"]
    try:
        got = pb.run()
    finally:
        pb.free()
    for b in range(2):
        _check(got[b].ravel(), pb.ref[b].ravel(), b)


# ----------------------------------------------------------- cache write path --

ALL = list(va.Fmt)


def _special_rows(rng, shape):
    x = rng.standard_normal(shape).astype(np.float32) * rng.choice([1e-3, 1.0, 40.0], shape)
    flat = x.reshape(-1, 32)
    flat[0] = 0.0                                              # all-zero group: scale 1, codes 0
    flat[1] = np.float32(6.5e-6)                               # fp16-subnormal scale
    flat[2, :4] = [3.5, -3.5, 2.5, 127.0]                      # exact .5 ties after division
    return x.astype(np.float16)


# f16 formats have no scales: one G for them
@pytest.mark.parametrize("fmt,G", [(f, G) for f in ALL for G in (32, 64) if va.fmt_bits(f) != 16 or G == 32],
                         ids=lambda x: x.label if isinstance(x, va.Fmt) else str(x))
def test_append_is_bit_exact(fmt, G):
    rng = np.random.default_rng(G + int(fmt))
    B, Hkv, D, P, n = 3, 2, 128, 16, 37
    start = np.array([0, 5, 30], np.int32)
    npg = 8
    table = rng.permutation(B * npg + 2)[:B * npg].reshape(B, npg).astype(np.int32)
    table[2, 4] = 10_000                         # sequence 2 crosses into an invalid page at 64
    num_pages = B * npg + 2
    rb = va.row_bytes(fmt, D)
    quant = va.fmt_bits(fmt) != 16
    pool = np.full((num_pages, Hkv, P, rb), 0xA5, np.uint8)
    spool = np.full((num_pages, Hkv, P, D // G), 0x5A5A, np.uint16)
    x = _special_rows(rng, (B, Hkv, n, D))
    shape = va.PagedShape(B, Hkv, Hkv, D, G, P, npg, num_pages, 0)
    print(f"append {fmt.label} G={G}", flush=True)
    dx, dst, dtab = (va.DeviceBuffer.from_array(a) for a in (x.view(np.uint16), start, table))
    dpool, dsp = va.DeviceBuffer.from_array(pool), va.DeviceBuffer.from_array(spool)
    try:
        va.append_kv(fmt, dx.ptr, n, dst.ptr, dtab.ptr, shape, dpool.ptr, dsp.ptr if quant else 0)
        va.sync()
        got = dpool.download(np.uint8).reshape(pool.shape)
        gots = dsp.download(np.uint16).reshape(spool.shape)
    finally:
        for d in (dx, dst, dtab, dpool, dsp):
            d.free()
    want, wants = pool.copy(), spool.copy()
    for b in range(B):
        for r in range(n):
            p = int(start[b]) + r
            pi = p // P
            if pi >= npg or not (0 <= table[b, pi] < num_pages):
                continue                          # not written
            for h in range(Hkv):
                row = x[b, h, r].astype(np.float32)
                if quant:
                    data, sc = oracle.quantize(row, D, G, va.fmt_bits(fmt))
                    want[table[b, pi], h, p % P] = data
                    wants[table[b, pi], h, p % P] = sc
                else:
                    want[table[b, pi], h, p % P] = x[b, h, r].view(np.uint8)
    np.testing.assert_array_equal(got, want)
    if quant:
        np.testing.assert_array_equal(gots, wants)


@pytest.mark.parametrize("fmt", TILED, ids=lambda f: f.label)
def test_append_then_decode(fmt):
    """Build each sequence's cache by appends (one row per call, then chunks),
    then decode the batch: equals the reference over the oracle's quantization
    of the same rows."""
    rng = np.random.default_rng(int(fmt))
    B, Hq, Hkv, D, G, P = 2, 8, 2, 128, 32, 64
    lens = [130, 77]
    npg = 4
    num_pages = B * npg
    table = rng.permutation(num_pages).reshape(B, npg).astype(np.int32)
    rb = va.row_bytes(fmt, D)
    quant = va.fmt_bits(fmt) != 16
    rows = {t: rng.standard_normal((B, Hkv, max(lens), D)).astype(np.float16) for t in "kv"}
    shape = va.PagedShape(B, Hq, Hkv, D, G, P, npg, num_pages, max(lens))
    pools = {t: va.DeviceBuffer(num_pages * Hkv * P * rb) for t in "kv"}
    spools = {t: va.DeviceBuffer(max(1, num_pages * Hkv * P * (D // G) * 2)) for t in "kv"}
    dtab = va.DeviceBuffer.from_array(table)
    q = batch_util.queries(B * Hq, D, 99).reshape(B, Hq, D)
    extra = []
    try:
        for t in "kv":
            # the first 10 positions one row per call, the rest in chunks of 37
            pos = 0
            while pos < max(lens):
                n = 1 if pos < 10 else min(37, max(lens) - pos)
                xs = np.ascontiguousarray(rows[t][:, :, pos:pos + n])
                dx = va.DeviceBuffer.from_array(xs.view(np.uint16))
                dst = va.DeviceBuffer.from_array(np.full(B, pos, np.int32))
                extra += [dx, dst]
                va.append_kv(fmt, dx.ptr, n, dst.ptr, dtab.ptr, shape, pools[t].ptr,
                             spools[t].ptr if quant else 0)
                pos += n
        out = va.DeviceBuffer(B * Hq * D * 2)
        S = va.pick_splits_paged(fmt, shape)
        ws = va.DeviceBuffer(va.ws_bytes(B * Hq, D, S))
        dq = va.DeviceBuffer.from_array(q)
        dl = va.DeviceBuffer.from_array(np.asarray(lens, np.int32))
        extra += [out, ws, dq, dl]
        pb = va.PagedBufs(K=pools["k"].ptr, V=pools["v"].ptr,
                          scK=spools["k"].ptr if quant else 0, scV=spools["v"].ptr if quant else 0,
                          block_table=dtab.ptr, seq_lens=dl.ptr, q=dq.ptr, out=out.ptr, ws=ws.ptr)
        va.decode_paged(fmt, pb, shape)
        va.sync()
        got = out.download(np.uint16).view(np.float16).astype(np.float32).reshape(B, Hq, D)
    finally:
        for d in list(pools.values()) + list(spools.values()) + [dtab] + extra:
            d.free()
    bits = va.fmt_bits(fmt)
    for b, L in enumerate(lens):
        deq = {}
        for t in "kv":
            x = rows[t][b, :, :L].astype(np.float32).reshape(-1)
            if quant:
                data, sc = oracle.quantize(x, D, G, bits)
                deq[t] = oracle.dequant(data, sc, Hkv * L, D, G, bits)
            else:
                deq[t] = x
        ref = batch.reference_gqa(deq["k"], deq["v"], q[b], Hq, Hkv, L, D)
        _check(got[b].ravel(), ref, (fmt.label, b))
