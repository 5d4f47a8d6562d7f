"""ctypes binding of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg and its after-timing output check, as the checker. The product (voltattn_amd) never
imports it. See oracle.hpp for what each function restates and how it is pinned.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"


def _load() -> C.CDLL:
    if not LIB_PATH.exists():
        subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return C.CDLL(str(LIB_PATH))


lib = _load()
_P, _I, _SZ, _U32 = C.c_void_p, C.c_int, C.c_size_t, C.c_uint32


def _sig(name, res, *args):
    fn = getattr(lib, name)
    fn.restype = res
    fn.argtypes = list(args)


_sig("oracle_f32_to_f16", C.c_uint16, C.c_float)
_sig("oracle_f16_to_f32", C.c_float, C.c_uint16)
_sig("oracle_f32_to_f16_array", None, _P, _SZ, _P)
_sig("oracle_mt_nth", _U32, _U32, _SZ)
_sig("oracle_mt_stream", None, _U32, _SZ, _P)
_sig("oracle_normal_stream", None, _U32, _SZ, _P)
_sig("oracle_selftest_seed", _U32, _I, _I, _I, _I)
_sig("oracle_draw", None, _U32, _I, _I, _I, _P, _P, _P)
_sig("oracle_packed_bytes", _SZ, _I, _SZ)
_sig("oracle_quantize", _I, _P, _SZ, _I, _I, _I, _P, _P)
_sig("oracle_codes", _I, _P, _SZ, _I, _P)
_sig("oracle_dequant", _I, _P, _P, _SZ, _I, _I, _I, _P)
_sig("oracle_reference", _I, _P, _P, _P, _I, _I, _I, _P)
_sig("oracle_reference_mt", _I, _P, _P, _P, _I, _I, _I, _I, _P)
_sig("oracle_split_attention", _I, _P, _P, _P, _I, _I, _I, _I, _P, _P, _P)
_sig("oracle_make_case", _I, _I, _I, _I, _I, _I, _U32, _P, _P, _P, _P, _P, _P, _P, _P)

# Selftest matrix of the reference (src/voltattn.cu:913-916): (H, L, D, S).
SELFTEST_SHAPES = [(8, 257, 128, 1), (8, 257, 128, 3), (2, 4096, 128, 5),
                   (40, 1000, 128, 2), (8, 129, 64, 1), (8, 513, 64, 4)]
# Formats in selftest order (src/voltattn.cu:918): name -> storage bits.
FORMATS = [("f16", 16), ("f16+", 16), ("q8", 8), ("q8+", 8), ("q4", 4), ("q4+", 4), ("q3+", 3)]


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


def f32_to_f16(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib.oracle_f32_to_f16_array(x.ctypes.data, x.size, out.ctypes.data)
    return out


def f16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    return np.array([lib.oracle_f16_to_f32(int(v)) for v in h.ravel()], np.float32).reshape(h.shape)


def mt_nth(seed: int, n: int) -> int:
    return int(lib.oracle_mt_nth(seed, n))


def mt_stream(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.uint32)
    lib.oracle_mt_stream(seed, n, out.ctypes.data)
    return out


def normal_stream(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib.oracle_normal_stream(seed, n, out.ctypes.data)
    return out


def selftest_seed(H: int, L: int, D: int, S: int) -> int:
    return int(lib.oracle_selftest_seed(H, L, D, S))


def draw(seed: int, H: int, L: int, D: int):
    n = H * L * D
    kx, vx, q = np.empty(n, np.float32), np.empty(n, np.float32), np.empty(H * D, np.uint16)
    lib.oracle_draw(seed, H, L, D, kx.ctypes.data, vx.ctypes.data, q.ctypes.data)
    return kx, vx, q


def packed_bytes(bits: int, n: int) -> int:
    return int(lib.oracle_packed_bytes(bits, n))


def quantize(x: np.ndarray, D: int, G: int, bits: int):
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    rows = x.size // D
    data = np.empty(packed_bytes(bits, x.size), np.uint8)
    scale = np.empty(rows * (D // G), np.uint16)
    if lib.oracle_quantize(x.ctypes.data, rows, D, G, bits, data.ctypes.data, scale.ctypes.data):
        raise ValueError("bad quantize arguments")
    return data, scale


def codes(data: np.ndarray, n: int, bits: int) -> np.ndarray:
    out = np.empty(n, np.int32)
    if lib.oracle_codes(np.ascontiguousarray(data).ctypes.data, n, bits, out.ctypes.data):
        raise ValueError("bad bits")
    return out


def dequant(data: np.ndarray, scale: np.ndarray, rows: int, D: int, G: int, bits: int) -> np.ndarray:
    out = np.empty(rows * D, np.float32)
    if lib.oracle_dequant(np.ascontiguousarray(data).ctypes.data,
                          np.ascontiguousarray(scale).ctypes.data, rows, D, G, bits, out.ctypes.data):
        raise ValueError("bad dequant arguments")
    return out


def reference(kd, vd, q, H: int, L: int, D: int, threads: int = 1) -> np.ndarray:
    kd = np.ascontiguousarray(kd, np.float32)
    vd = np.ascontiguousarray(vd, np.float32)
    q = np.ascontiguousarray(q, np.uint16)
    out = np.empty(H * D, np.float32)
    if threads > 1:
        rc = lib.oracle_reference_mt(kd.ctypes.data, vd.ctypes.data, q.ctypes.data, H, L, D,
                                     threads, out.ctypes.data)
    else:
        rc = lib.oracle_reference(kd.ctypes.data, vd.ctypes.data, q.ctypes.data, H, L, D,
                                  out.ctypes.data)
    if rc:
        raise ValueError("bad reference arguments")
    return out


def split_attention(kd, vd, q, H: int, L: int, D: int, S: int):
    """Returns (out[H*D], lse[H,S] natural log, avg[H,S,D] = o_s / l_s)."""
    kd = np.ascontiguousarray(kd, np.float32)
    vd = np.ascontiguousarray(vd, np.float32)
    q = np.ascontiguousarray(q, np.uint16)
    out = np.empty(H * D, np.float32)
    lse = np.empty((H, S), np.float64)
    avg = np.empty((H, S, D), np.float64)
    if lib.oracle_split_attention(kd.ctypes.data, vd.ctypes.data, q.ctypes.data, H, L, D, S,
                                  out.ctypes.data, lse.ctypes.data, avg.ctypes.data):
        raise ValueError("bad split arguments")
    return out, lse, avg


def make_case(bits: int, H: int, L: int, D: int, G: int, seed: int, want_dequant: bool = True) -> dict:
    """Inputs + double reference of one selftest-style case (run_case, src/voltattn.cu:838-861)."""
    n = H * L * D
    pay = packed_bytes(bits, n)
    c = {
        "kd": np.empty(n, np.float32) if want_dequant else None,
        "vd": np.empty(n, np.float32) if want_dequant else None,
        "q": np.empty(H * D, np.uint16),
        "kpay": np.empty(pay, np.uint8),
        "vpay": np.empty(pay, np.uint8),
        "ksc": np.empty(n // G, np.uint16) if bits != 16 else None,
        "vsc": np.empty(n // G, np.uint16) if bits != 16 else None,
        "ref": np.empty(H * D, np.float32),
    }
    rc = lib.oracle_make_case(bits, H, L, D, G, seed, _ptr(c["kd"]), _ptr(c["vd"]), _ptr(c["q"]),
                              _ptr(c["kpay"]), _ptr(c["vpay"]), _ptr(c["ksc"]), _ptr(c["vsc"]),
                              _ptr(c["ref"]))
    if rc:
        raise ValueError("bad case arguments")
    c.update(bits=bits, H=H, L=L, D=D, G=G, seed=seed)
    return c


def gate(got: np.ndarray, ref: np.ndarray) -> tuple[bool, float]:
    """The reference's pass rule |got - ref| <= 3e-3 + 2e-2|ref| (src/voltattn.cu:896-904)."""
    g = np.asarray(got, np.float64)
    r = np.asarray(ref, np.float64)
    err = np.abs(g - r)
    return bool(np.all(err <= 3e-3 + 2e-2 * np.abs(r))), float(err.max()) if err.size else 0.0
