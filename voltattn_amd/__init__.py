"""voltattn_amd — MI355X (gfx950) fused dequant + decode attention.

Python mirror of kamilch1k/voltattn's host interface over the C ABI of
``include/voltattn.h`` (``libvoltattn_hip.so``, built in-tree by
``python voltattn_amd/build.py``):

* :class:`Fmt` — the reference's ``enum class Fmt`` (src/voltattn.cu:676);
* :class:`DeviceBufs` — ``struct DeviceBufs`` (src/voltattn.cu:796-801);
* :func:`launch` — ``launch(f, b, H, L, D, S)`` (src/voltattn.cu:803-835), with
  the group size ``G`` added (the reference fixes 64, src/voltattn.cu:60).

Errors raise :class:`VAError` carrying the library's status code and message,
where the reference exits through ``CUDA_CHECK`` (src/voltattn.cu:49-58). There
is no fallback: without the built HIP library this package does not import.
"""
from __future__ import annotations

import ctypes as C
import enum
import os
from dataclasses import dataclass
from pathlib import Path

import numpy as np

__all__ = [
    "Fmt", "DeviceBufs", "VAError", "launch", "decode_splits", "merge", "ws_bytes",
    "payload_bytes", "scale_bytes", "split_chunk", "pick_splits", "quantize", "dequantize", "f32_to_f16",
    "fill_normal", "probe_read", "probe_digest", "probe_read_sized", "merge_faults", "device_info", "device_count", "DeviceBuffer", "Event",
    "Stream", "Graph", "sync", "lib", "LIB_PATH", "fmt_bits", "is_f16", "check",
    "PagedShape", "PagedBufs", "decode_gqa", "pick_splits_gqa", "decode_paged",
    "pick_splits_paged", "page_bytes", "page_scale_bytes", "append_kv", "row_bytes",
]

LIB_PATH = Path(__file__).resolve().parent / "libvoltattn_hip.so"
if not LIB_PATH.exists():
    raise ImportError(
        f"{LIB_PATH} is not built; run `python voltattn_amd/build.py` (needs hipcc for gfx950)")


def _bind_torch_hip_runtime() -> None:
    """Load PyTorch-ROCm's own HIP runtime first, so this library binds to it.

    A process holds one HIP runtime per loaded copy of libamdhip64; PyTorch-ROCm
    ships its own and loads it by path. When this library has already brought in
    the system ROCm runtime and initialised it, torch's later device init fails
    ("No HIP GPUs are available"). Importing torch first avoids that by itself
    (the library then binds to torch's already-loaded runtime by soname);
    VOLTATTN_HIP_RUNTIME=torch does the same without importing torch."""
    import importlib.util
    spec = importlib.util.find_spec("torch")
    if spec is None or not spec.submodule_search_locations:
        raise ImportError("VOLTATTN_HIP_RUNTIME=torch but PyTorch is not installed")
    rt = Path(list(spec.submodule_search_locations)[0]) / "lib" / "libamdhip64.so"
    if not rt.exists():
        raise ImportError(f"VOLTATTN_HIP_RUNTIME=torch but {rt} does not exist (not a ROCm build of torch?)")
    C.CDLL(str(rt), mode=C.RTLD_GLOBAL)


if os.environ.get("VOLTATTN_HIP_RUNTIME", "system") == "torch":
    _bind_torch_hip_runtime()
lib = C.CDLL(str(LIB_PATH))

_P, _I, _SZ, _U64 = C.c_void_p, C.c_int, C.c_size_t, C.c_uint64


class _Bufs(C.Structure):
    _fields_ = [("k", _P), ("v", _P), ("sk", _P), ("sv", _P), ("q", _P), ("out", _P), ("ws", _P)]


class _PagedShape(C.Structure):
    _fields_ = [("B", _I), ("Hq", _I), ("Hkv", _I), ("D", _I), ("G", _I), ("page_rows", _I),
                ("max_pages", _I), ("num_pages", _I), ("max_seq_len", _I)]


class _PagedBufs(C.Structure):
    _fields_ = [("k", _P), ("v", _P), ("sk", _P), ("sv", _P), ("block_table", _P),
                ("seq_lens", _P), ("q", _P), ("out", _P), ("ws", _P)]


class _DevInfo(C.Structure):
    _fields_ = [("name", C.c_char * 256), ("arch", C.c_char * 64), ("compute_units", _I),
                ("clock_khz", _I), ("mem_clock_khz", _I), ("mem_bus_bits", _I),
                ("total_mem", _SZ), ("l2_bytes", _SZ)]


def _sig(name, res, *args):
    fn = getattr(lib, name)
    fn.restype = res
    fn.argtypes = list(args)
    return fn


_sig("va_decode", _I, _I, C.POINTER(_Bufs), _I, _I, _I, _I, _I, _P)
_sig("va_decode_splits", _I, _I, C.POINTER(_Bufs), _I, _I, _I, _I, _I, _P)
_sig("va_merge", _I, _P, _P, _I, _I, _I, _P)
_sig("va_merge_faults", _I, _P, C.POINTER(C.c_uint))
_sig("va_decode_noalloc", _I, _I, C.POINTER(_Bufs), _I, _I, _I, _I, _I, _P)
_sig("va_ws_bytes", _SZ, _I, _I, _I)
_sig("va_payload_bytes", _SZ, _I, _I, _I, _I)
_sig("va_scale_bytes", _SZ, _I, _I, _I, _I, _I)
_sig("va_split_chunk", _I, _I, _I)
_sig("va_pick_splits", _I, _I, _I, _I, _I, C.POINTER(_I))
_sig("va_fmt_name", C.c_char_p, _I)
_sig("va_quantize", _I, _I, _I, _P, _SZ, _I, _P, _P, _P)
_sig("va_dequantize", _I, _I, _I, _P, _P, _SZ, _I, _P, _P)
_sig("va_f32_to_f16", _I, _P, _SZ, _P, _P)
_sig("va_fill_normal", _I, _P, _SZ, _U64, _P)
_sig("va_probe_read", _I, _SZ, _I, C.POINTER(C.c_double))
_sig("va_probe_launch", _I, _I, C.POINTER(C.c_double))
_sig("va_probe_digest", _I, _P, _SZ, _I, _I, _I, C.POINTER(C.c_uint32), C.POINTER(_U64), C.POINTER(_SZ))
_sig("va_probe_read_sized", _I, _SZ, _SZ, _I, C.POINTER(C.c_double), C.POINTER(C.c_double))
_sig("va_decode_gqa", _I, _I, C.POINTER(_Bufs), _I, _I, _I, _I, _I, _I, _P)
_sig("va_pick_splits_gqa", _I, _I, _I, _I, _I, _I, C.POINTER(_I))
_sig("va_decode_paged", _I, _I, C.POINTER(_PagedBufs), C.POINTER(_PagedShape), _I, _P)
_sig("va_pick_splits_paged", _I, _I, C.POINTER(_PagedShape), C.POINTER(_I))
_sig("va_page_bytes", _SZ, _I, _I, _I, _I)
_sig("va_page_scale_bytes", _SZ, _I, _I, _I, _I, _I)
_sig("va_append_kv", _I, _I, _P, _I, _P, _P, C.POINTER(_PagedShape), _P, _P, _P)
_sig("va_device_count", _I, C.POINTER(_I))
_sig("va_set_device", _I, _I)
_sig("va_device_info", _I, C.POINTER(_DevInfo))
_sig("va_malloc", _I, C.POINTER(_P), _SZ)
_sig("va_free", _I, _P)
_sig("va_memcpy_h2d", _I, _P, _P, _SZ)
_sig("va_memcpy_d2h", _I, _P, _P, _SZ)
_sig("va_memcpy_d2d", _I, _P, _P, _SZ, _P)
_sig("va_memset", _I, _P, _I, _SZ)
_sig("va_sync", _I)
_sig("va_stream_create", _I, C.POINTER(_P))
_sig("va_stream_destroy", _I, _P)
_sig("va_stream_sync", _I, _P)
_sig("va_stream_release", _I, _P)
_sig("va_capture_release", _I, C.c_ulonglong)
_sig("va_event_create", _I, C.POINTER(_P))
_sig("va_event_destroy", _I, _P)
_sig("va_event_record", _I, _P, _P)
_sig("va_event_sync", _I, _P)
_sig("va_event_elapsed_ms", _I, _P, _P, C.POINTER(C.c_float))
_sig("va_graph_begin", _I, _P)
_sig("va_graph_end", _I, _P, C.POINTER(_P))
_sig("va_graph_launch", _I, _P, _P)
_sig("va_graph_destroy", _I, _P)
_sig("va_last_error", C.c_char_p)
_sig("va_abi_version", _I)


class VAError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"voltattn error {code}: {msg}")
        self.code = code


def check(rc: int) -> None:
    if rc != 0:
        raise VAError(rc, lib.va_last_error().decode(errors="replace"))


class Fmt(enum.IntEnum):
    """src/voltattn.cu:676 — F16, F16M (f16+), Q8, Q8M (q8+), Q4, Q4M (q4+), Q3M (q3+)."""
    F16 = 0
    F16M = 1
    Q8 = 2
    Q8M = 3
    Q4 = 4
    Q4M = 5
    Q3M = 6

    @property
    def label(self) -> str:
        return lib.va_fmt_name(int(self)).decode()

    @classmethod
    def parse(cls, s: str) -> "Fmt":
        for f in cls:
            if f.label == s.strip() or f.name == s.strip().upper():
                return f
        raise ValueError(f"unknown format {s!r}")


def fmt_bits(f: Fmt) -> int:
    return {Fmt.F16: 16, Fmt.F16M: 16, Fmt.Q8: 8, Fmt.Q8M: 8, Fmt.Q4: 4, Fmt.Q4M: 4, Fmt.Q3M: 3}[Fmt(f)]


def is_f16(f: Fmt) -> bool:
    return fmt_bits(f) == 16


@dataclass
class DeviceBufs:
    """src/voltattn.cu:796-801. Device pointers as ints (0 = NULL)."""
    K: int = 0
    V: int = 0
    scK: int = 0
    scV: int = 0
    q: int = 0
    out: int = 0
    ws: int = 0

    def _c(self) -> _Bufs:
        return _Bufs(self.K or None, self.V or None, self.scK or None, self.scV or None,
                     self.q or None, self.out or None, self.ws or None)


def _stream(stream) -> int | None:
    if stream is None:
        return None
    return stream.handle if isinstance(stream, Stream) else int(stream)


def launch(f: Fmt, b: DeviceBufs, H: int, L: int, D: int, S: int, G: int = 64, stream=None) -> None:
    """One decode step (both passes), asynchronous on `stream`."""
    cb = b._c()
    check(lib.va_decode(int(f), C.byref(cb), H, L, D, G, S, _stream(stream)))


def decode_splits(f: Fmt, b: DeviceBufs, H: int, L: int, D: int, S: int, G: int = 64,
                  stream=None) -> None:
    """First pass only: S partials (m, l, o[D]) per head into b.ws (m in log2 units)."""
    cb = b._c()
    check(lib.va_decode_splits(int(f), C.byref(cb), H, L, D, G, S, _stream(stream)))


def merge(ws: int, out: int, H: int, D: int, S: int, stream=None) -> None:
    check(lib.va_merge(ws, out, H, D, S, _stream(stream)))


def merge_faults(stream=None) -> int:
    """Fused merges on the current device that gave up waiting for a partial since
    the previous query (their outputs are NaN); raises VAError (VA_ELOST = 7) if any.
    Synchronizes `stream` first."""
    n = C.c_uint(0)
    check(lib.va_merge_faults(_stream(stream), C.byref(n)))
    return n.value


def decode_gqa(f: Fmt, b: DeviceBufs, Hq: int, Hkv: int, L: int, D: int, S: int = 0, G: int = 64,
               stream=None) -> None:
    """One sequence, Hq query heads over Hkv KV heads (query head h reads KV head
    h // (Hq // Hkv)); q/out are [Hq][D], K/V [Hkv][L][row]. S = 0 picks it."""
    cb = b._c()
    check(lib.va_decode_gqa(int(f), C.byref(cb), Hq, Hkv, L, D, G, S, _stream(stream)))


def pick_splits_gqa(f: Fmt, Hq: int, Hkv: int, L: int, D: int) -> int:
    s = _I(0)
    check(lib.va_pick_splits_gqa(int(f), Hq, Hkv, L, D, C.byref(s)))
    return s.value


@dataclass
class PagedShape:
    """va_paged_shape: a batch of B sequences over a page pool of num_pages pages,
    each holding [Hkv][page_rows][row] (+ [Hkv][page_rows][D/G] fp16 scales)."""
    B: int
    Hq: int
    Hkv: int
    D: int
    G: int
    page_rows: int
    max_pages: int
    num_pages: int
    max_seq_len: int

    def _c(self) -> _PagedShape:
        return _PagedShape(self.B, self.Hq, self.Hkv, self.D, self.G, self.page_rows,
                           self.max_pages, self.num_pages, self.max_seq_len)


@dataclass
class PagedBufs:
    """va_paged_bufs: device pointers as ints (0 = NULL)."""
    K: int = 0
    V: int = 0
    scK: int = 0
    scV: int = 0
    block_table: int = 0
    seq_lens: int = 0
    q: int = 0
    out: int = 0
    ws: int = 0

    def _c(self) -> _PagedBufs:
        return _PagedBufs(self.K or None, self.V or None, self.scK or None, self.scV or None,
                          self.block_table or None, self.seq_lens or None, self.q or None,
                          self.out or None, self.ws or None)


def decode_paged(f: Fmt, b: PagedBufs, shape: PagedShape, S: int = 0, stream=None) -> None:
    """One decode step of every sequence of a paged batch (q/out [B][Hq][D])."""
    cb, cs = b._c(), shape._c()
    check(lib.va_decode_paged(int(f), C.byref(cb), C.byref(cs), S, _stream(stream)))


def pick_splits_paged(f: Fmt, shape: PagedShape) -> int:
    s = _I(0)
    cs = shape._c()
    check(lib.va_pick_splits_paged(int(f), C.byref(cs), C.byref(s)))
    return s.value


def page_bytes(f: Fmt, Hkv: int, page_rows: int, D: int) -> int:
    return lib.va_page_bytes(int(f), Hkv, page_rows, D)


def page_scale_bytes(f: Fmt, Hkv: int, page_rows: int, D: int, G: int) -> int:
    return lib.va_page_scale_bytes(int(f), Hkv, page_rows, D, G)


def append_kv(f: Fmt, x: int, n: int, start: int, block_table: int, shape: PagedShape, pages: int,
              scales: int = 0, stream=None) -> None:
    """Quantize-and-append n new fp16 rows per (sequence, KV head), x [B][Hkv][n][D],
    at positions start[b] + r of a paged cache."""
    cs = shape._c()
    check(lib.va_append_kv(int(f), x, n, start, block_table, C.byref(cs), pages, scales or None,
                           _stream(stream)))


def row_bytes(f: Fmt, D: int) -> int:
    return D * fmt_bits(f) // 8


def ws_bytes(H: int, D: int, S: int) -> int:
    return lib.va_ws_bytes(H, D, S)


def payload_bytes(f: Fmt, H: int, L: int, D: int) -> int:
    return lib.va_payload_bytes(int(f), H, L, D)


def scale_bytes(f: Fmt, H: int, L: int, D: int, G: int) -> int:
    return lib.va_scale_bytes(int(f), H, L, D, G)


def split_chunk(L: int, S: int) -> int:
    return lib.va_split_chunk(L, S)


def pick_splits(f: Fmt, H: int, L: int, D: int) -> int:
    s = _I(0)
    check(lib.va_pick_splits(int(f), H, L, D, C.byref(s)))
    return s.value


def quantize(bits: int, G: int, x: int, rows: int, D: int, packed: int, scales: int, stream=None) -> None:
    check(lib.va_quantize(bits, G, x, rows, D, packed, scales, _stream(stream)))


def dequantize(bits: int, G: int, packed: int, scales: int, rows: int, D: int, out: int, stream=None) -> None:
    """va_dequantize: packed codes + fp16 scales (device pointers) to fp32 out[rows][D]."""
    check(lib.va_dequantize(bits, G, packed, scales, rows, D, out, _stream(stream)))


def f32_to_f16(x: int, n: int, out: int, stream=None) -> None:
    check(lib.va_f32_to_f16(x, n, out, _stream(stream)))


def fill_normal(x: int, n: int, seed: int, stream=None) -> None:
    check(lib.va_fill_normal(x, n, seed, _stream(stream)))


def probe_read(nbytes: int, reps: int = 10) -> float:
    g = C.c_double(0.0)
    check(lib.va_probe_read(nbytes, reps, C.byref(g)))
    return g.value


def probe_digest(src: int, nbytes: int, form: int, grid: int, unroll: int):
    """va_probe_digest: one launch of read-probe form `form` (0 grid-stride,
    1 chunked) over device buffer `src`; returns (xor of every 16-byte word read
    as 16 bytes, number of 16-byte loads, bytes credited)."""
    x = (C.c_uint32 * 4)()
    n = _U64(0)
    b = _SZ(0)
    check(lib.va_probe_digest(src, nbytes, form, grid, unroll, x, C.byref(n), C.byref(b)))
    import struct
    return struct.pack("<4I", *x), n.value, b.value


def probe_read_sized(nbytes: int, min_set: int = 2 << 30, launches: int = 50):
    """va_probe_read_sized: (us per launch, GB/s) of the chunked read of exactly
    `nbytes` per launch, back to back over copies spanning >= min_set bytes."""
    us = C.c_double(0.0)
    g = C.c_double(0.0)
    check(lib.va_probe_read_sized(nbytes, min_set, launches, C.byref(us), C.byref(g)))
    return us.value, g.value


def probe_launch(launches: int = 2000) -> float:
    """Microseconds per back-to-back launch of an empty kernel on the decode grid."""
    us = C.c_double(0.0)
    check(lib.va_probe_launch(launches, C.byref(us)))
    return us.value


def device_count() -> int:
    n = _I(0)
    rc = lib.va_device_count(C.byref(n))
    return n.value if rc == 0 else 0


def device_info() -> dict:
    d = _DevInfo()
    check(lib.va_device_info(C.byref(d)))
    return {"name": d.name.decode(), "arch": d.arch.decode(), "compute_units": d.compute_units,
            "clock_khz": d.clock_khz, "mem_clock_khz": d.mem_clock_khz,
            "mem_bus_bits": d.mem_bus_bits, "total_mem": d.total_mem, "l2_bytes": d.l2_bytes}


def sync() -> None:
    check(lib.va_sync())


class DeviceBuffer:
    """Owned device allocation (va_malloc/va_free)."""

    def __init__(self, nbytes: int):
        p = _P()
        check(lib.va_malloc(C.byref(p), max(1, int(nbytes))))
        self.ptr = int(p.value)
        self.nbytes = int(nbytes)

    @classmethod
    def from_array(cls, arr: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(arr)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, arr: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(arr)
        if offset + a.nbytes > self.nbytes:
            raise ValueError("upload exceeds buffer")
        check(lib.va_memcpy_h2d(self.ptr + offset, a.ctypes.data, a.nbytes))

    def download(self, dtype, count: int | None = None, offset: int = 0) -> np.ndarray:
        dt = np.dtype(dtype)
        n = (self.nbytes - offset) // dt.itemsize if count is None else int(count)
        out = np.empty(n, dtype=dt)
        check(lib.va_memcpy_d2h(out.ctypes.data, self.ptr + offset, out.nbytes))
        return out

    def zero(self) -> None:
        check(lib.va_memset(self.ptr, 0, self.nbytes))

    def free(self) -> None:
        if self.ptr:
            check(lib.va_free(self.ptr))
            self.ptr = 0

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.free()


class Stream:
    def __init__(self):
        p = _P()
        check(lib.va_stream_create(C.byref(p)))
        self.handle = int(p.value)

    def synchronize(self) -> None:
        check(lib.va_stream_sync(self.handle))

    def destroy(self) -> None:
        if self.handle:
            check(lib.va_stream_destroy(self.handle))
            self.handle = 0


class Event:
    def __init__(self):
        p = _P()
        check(lib.va_event_create(C.byref(p)))
        self.handle = int(p.value)

    def record(self, stream=None) -> None:
        check(lib.va_event_record(self.handle, _stream(stream)))

    def synchronize(self) -> None:
        check(lib.va_event_sync(self.handle))

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float(0.0)
        check(lib.va_event_elapsed_ms(self.handle, end.handle, C.byref(ms)))
        return float(ms.value)

    def destroy(self) -> None:
        if self.handle:
            check(lib.va_event_destroy(self.handle))
            self.handle = 0


class Graph:
    """A captured launch sequence: `with Graph.capture(stream) as g: ...` then g.launch(stream)."""

    def __init__(self, handle: int):
        self.handle = handle

    @classmethod
    def capture(cls, stream: "Stream"):
        return _Capture(stream)

    def launch(self, stream=None) -> None:
        check(lib.va_graph_launch(self.handle, _stream(stream)))

    def destroy(self) -> None:
        if self.handle:
            check(lib.va_graph_destroy(self.handle))
            self.handle = 0


class _Capture:
    def __init__(self, stream: "Stream"):
        self.stream = stream
        self.graph: Graph | None = None

    def __enter__(self) -> "_Capture":
        check(lib.va_graph_begin(_stream(self.stream)))
        return self

    def __exit__(self, exc_type, exc, tb):
        h = _P()
        rc = lib.va_graph_end(_stream(self.stream), C.byref(h))
        if exc_type is None:
            check(rc)
            self.graph = Graph(int(h.value))
        return False
