"""The grouped-query, paged and append entry points of the C ABI without a GPU:
sizes, and invalid arguments rejected with the documented status codes before
any device access (fake pointers below are never dereferenced)."""
import ctypes as C

import pytest

import voltattn_amd as va

VA_OK, VA_EINVAL, VA_EALIGN, VA_ENULL, VA_ERANGE = 0, 1, 2, 3, 4


def _bufs(k=0x1000, v=0x2000, sk=0x3000, sv=0x4000, q=0x5000, out=0x6000, ws=0x7000):
    return va._Bufs(k, v, sk, sv, q, out, ws)


def _pbufs(**kw):
    p = dict(k=0x10000, v=0x20000, sk=0x30000, sv=0x40000, block_table=0x50000,
             seq_lens=0x60000, q=0x70000, out=0x80000, ws=0x90000)
    p.update(kw)
    return va._PagedBufs(p["k"], p["v"], p["sk"], p["sv"], p["block_table"], p["seq_lens"],
                         p["q"], p["out"], p["ws"])


def _shape(**kw):
    s = dict(B=4, Hq=32, Hkv=8, D=128, G=32, page_rows=256, max_pages=64, num_pages=256,
             max_seq_len=16384)
    s.update(kw)
    return va._PagedShape(s["B"], s["Hq"], s["Hkv"], s["D"], s["G"], s["page_rows"],
                          s["max_pages"], s["num_pages"], s["max_seq_len"])


def test_page_sizes():
    assert va.page_bytes(va.Fmt.Q8M, 8, 256, 128) == 8 * 256 * 128
    assert va.page_bytes(va.Fmt.Q4M, 8, 256, 128) == 8 * 256 * 64
    assert va.page_bytes(va.Fmt.Q3M, 8, 256, 128) == 8 * 256 * 48
    assert va.page_bytes(va.Fmt.F16M, 8, 256, 64) == 8 * 256 * 128
    assert va.page_scale_bytes(va.Fmt.Q8M, 8, 256, 128, 32) == 8 * 256 * 4 * 2
    assert va.page_scale_bytes(va.Fmt.F16M, 8, 256, 128, 32) == 0
    assert va.page_bytes(va.Fmt.Q8M, 0, 256, 128) == 0


@pytest.mark.parametrize("fmt,Hq,Hkv,L,D,G,S,code,msg", [
    (va.Fmt.Q8, 8, 2, 100, 128, 32, 0, VA_EINVAL, "tiled format"),       # naive formats: no GQA
    (va.Fmt.Q8M, 9, 2, 100, 128, 32, 0, VA_EINVAL, "multiple of Hkv"),
    (va.Fmt.Q8M, 8, 0, 100, 128, 32, 0, VA_EINVAL, "multiple of Hkv"),
    (va.Fmt.Q8M, 8, 2, 100, 96, 32, 0, VA_EINVAL, "D must be"),
    (va.Fmt.Q8M, 8, 2, 0, 128, 32, 0, VA_EINVAL, "L must be"),
    (va.Fmt.Q8M, 8, 2, 100, 128, 32, -1, VA_EINVAL, "S must be"),
    (va.Fmt.Q4M, 8, 2, 100, 128, 16, 0, VA_EINVAL, "G must be"),
    (va.Fmt.Q8M, 8, 2, 1 << 30, 128, 32, 0, VA_ERANGE, "2^31"),
])
def test_gqa_rejects(fmt, Hq, Hkv, L, D, G, S, code, msg):
    b = _bufs()
    assert va.lib.va_decode_gqa(int(fmt), C.byref(b), Hq, Hkv, L, D, G, S, None) == code
    assert msg in va.lib.va_last_error().decode()


@pytest.mark.parametrize("field", ["k", "q", "out", "ws", "sv"])
def test_gqa_null_buffers(field):
    b = _bufs(**{field: 0})
    assert va.lib.va_decode_gqa(int(va.Fmt.Q8M), C.byref(b), 8, 2, 100, 128, 32, 0, None) == VA_ENULL


@pytest.mark.parametrize("shape,code,msg", [
    (dict(page_rows=48), VA_EINVAL, "power of two"),
    (dict(page_rows=32), VA_EINVAL, "power of two"),          # below the 64-row wave tile
    (dict(Hq=30), VA_EINVAL, "multiple of Hkv"),
    (dict(B=0), VA_EINVAL, "B and Hkv"),
    (dict(max_seq_len=64 * 256 + 1), VA_EINVAL, "max_seq_len"),
    (dict(max_seq_len=-1), VA_EINVAL, "max_seq_len"),
    (dict(D=80), VA_EINVAL, "D must be"),
    (dict(G=48), VA_EINVAL, "G must be"),
    (dict(num_pages=0), VA_EINVAL, "num_pages"),
    (dict(max_pages=1 << 20, page_rows=1 << 12), VA_ERANGE, "2^31"),
])
def test_paged_shape_rejects(shape, code, msg):
    b, s = _pbufs(), _shape(**shape)
    assert va.lib.va_decode_paged(int(va.Fmt.Q8M), C.byref(b), C.byref(s), 0, None) == code
    assert msg in va.lib.va_last_error().decode()


def test_paged_needs_tiled_format():
    b, s = _pbufs(), _shape()
    assert va.lib.va_decode_paged(int(va.Fmt.Q4), C.byref(b), C.byref(s), 0, None) == VA_EINVAL


@pytest.mark.parametrize("field,code", [
    ("block_table", VA_ENULL), ("seq_lens", VA_ENULL), ("k", VA_ENULL), ("ws", VA_ENULL),
    ("sk", VA_ENULL), ("q", VA_ENULL),
])
def test_paged_null_buffers(field, code):
    b, s = _pbufs(**{field: 0}), _shape()
    assert va.lib.va_decode_paged(int(va.Fmt.Q8M), C.byref(b), C.byref(s), 0, None) == code


@pytest.mark.parametrize("field,ptr", [("k", 0x10004), ("q", 0x70008), ("sk", 0x30002),
                                       ("block_table", 0x50002), ("seq_lens", 0x60001)])
def test_paged_alignment(field, ptr):
    b, s = _pbufs(**{field: ptr}), _shape()
    assert va.lib.va_decode_paged(int(va.Fmt.Q8M), C.byref(b), C.byref(s), 0, None) == VA_EALIGN


def test_paged_split_spanning_too_many_pages():
    # page_rows 64, one split over 128K positions would span 2049 pages
    b, s = _pbufs(), _shape(B=1, page_rows=64, max_pages=4096, num_pages=4096, max_seq_len=131072)
    assert va.lib.va_decode_paged(int(va.Fmt.Q8M), C.byref(b), C.byref(s), 1, None) == VA_EINVAL
    assert "raise S" in va.lib.va_last_error().decode()


def test_pick_splits_paged_keeps_splits_within_page_limit():
    s = _shape(B=1, Hq=8, Hkv=8, page_rows=64, max_pages=4096, num_pages=4096, max_seq_len=262144)
    out = C.c_int(0)
    assert va.lib.va_pick_splits_paged(int(va.Fmt.Q8M), C.byref(s), C.byref(out)) == VA_OK
    S = out.value
    chunk = -(-262144 // S)
    assert chunk // 64 + 2 <= 1024


def test_append_rejects():
    s = _shape()
    ok = dict(fmt=int(va.Fmt.Q8M), x=0x1000, n=1, start=0x2000, table=0x3000, pages=0x4000, scales=0x5000)

    def call(**kw):
        p = dict(ok)
        p.update(kw)
        return va.lib.va_append_kv(p["fmt"], p["x"], p["n"], p["start"], p["table"], C.byref(s),
                                   p["pages"], p["scales"], None)

    assert call(n=-1) == VA_EINVAL
    assert call(n=0) == VA_OK                      # nothing to write: no launch
    assert call(x=None) == VA_ENULL
    assert call(scales=None) == VA_ENULL
    assert call(fmt=int(va.Fmt.F16M), scales=None, pages=0x4004) == VA_EALIGN   # f16 rows are 16-byte copies
    assert call(x=0x1008) == VA_EALIGN
    assert call(fmt=9) == VA_EINVAL
