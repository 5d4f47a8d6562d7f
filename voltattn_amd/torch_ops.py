"""PyTorch-ROCm binding: ``torch.ops.voltattn.*`` custom ops over the C ABI.

Importing this module registers

* ``voltattn::decode(q, k, v, k_scale, v_scale, fmt, group, splits) -> out``
  — one decode step (va_decode; the reference's launch(), src/voltattn.cu:803-835);
* ``voltattn::decode_gqa(...)`` — Hq query heads over Hkv KV heads (va_decode_gqa);
* ``voltattn::decode_paged(...)`` — a batch over a page pool (va_decode_paged);
* ``voltattn::append_kv(...)`` — quantize-and-append new rows (va_append_kv; mutates the pools);
* ``voltattn::quantize(x, bits, group) -> (packed, scales)`` (va_quantize; the reference's
  quantize(), src/voltattn.cu:705-745);
* ``voltattn::dequantize(packed, scales, bits, group) -> x`` (va_dequantize; the reference's
  dq(), src/voltattn.cu:747-767, over whole rows: fp32 [..., D]).

Tensors keep the C ABI's layouts (include/voltattn.h): q/out fp16 [.., H, D];
quantized K/V payload uint8 [.., L, row bytes]; f16 K/V fp16 [.., L, D]; scales
fp16 [.., L, D/G]. Every op runs asynchronously on torch's current HIP stream
and fails loudly on invalid input: the shapes and dtypes of every tensor are
checked against (fmt, D, G) before the C ABI is called, in the real and the
fake (meta) implementation alike (RuntimeError), and the library's own checks
raise with its message. There is no CPU fallback: the tensors must live on a
gfx950 device. Each op has a fake implementation, so shapes propagate under
torch.compile.
"""
from __future__ import annotations

import ctypes as C
from typing import Optional

import torch

from . import (Fmt, _Bufs, _PagedBufs, _PagedShape, check, fmt_bits, lib, ws_bytes)

__all__ = ["decode", "decode_gqa", "decode_paged", "append_kv", "quantize", "dequantize"]


def _fmt(name: str) -> Fmt:
    return Fmt.parse(name)


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _stream(t: torch.Tensor):
    return torch.cuda.current_stream(t.device).cuda_stream


def _need_gpu(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError("voltattn ops need tensors on a gfx950 device (no CPU fallback)")
        if t is not None and not t.is_contiguous():
            raise RuntimeError("voltattn ops need contiguous tensors")


def _D_of(q: torch.Tensor) -> int:
    return int(q.shape[-1])


def _fail(msg: str):
    raise RuntimeError(f"voltattn: {msg}")


# The validators run in the real and the fake (meta) implementations alike.
# Sizes may be symbolic (torch.compile with dynamic shapes): they are compared
# with torch._check, which records a runtime assertion instead of fixing a
# size to its traced value, and are never converted with int() here, so a
# decode loop whose L grows does not recompile on every step. Only the head
# dimension D (64 or 128) and the group size decide which kernel runs.

def _check(cond, msg) -> None:
    torch._check(cond, lambda: f"voltattn: {msg()}")


def _expect(t: torch.Tensor, name: str, shape: tuple, dtype: torch.dtype) -> None:
    if t is None:
        _fail(f"{name} is required")
    if t.dim() != len(shape):
        _fail(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    for got, want in zip(t.shape, shape):
        _check(got == want, lambda: f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    if t.dtype != dtype:
        _fail(f"{name} has dtype {t.dtype}, expected {dtype}")


def _check_dg(f: Fmt, D, group: int) -> None:
    _check((D == 64) | (D == 128), lambda: f"D must be 64 or 128 (got {D})")
    if fmt_bits(f) != 16:
        if group not in (32, 64):
            _fail(f"group must be 32 or 64 (got {group})")
        _check(D >= group, lambda: f"group must be <= D (got {group}, D={D})")


def _row_shape(f: Fmt, D) -> tuple[tuple, torch.dtype]:
    """Trailing shape and dtype of one K/V row of format f: fp16 [D] for the f16
    formats, uint8 [row bytes] for the quantized ones."""
    if fmt_bits(f) == 16:
        return (D,), torch.float16
    return (D * fmt_bits(f) // 8,), torch.uint8


def _check_kv(f: Fmt, k, v, ks, vs, lead: tuple, D, group: int) -> None:
    """k, v [*lead, row]; scales fp16 [*lead, D/G] for quantized formats."""
    tail, dt = _row_shape(f, D)
    _expect(k, "k", lead + tail, dt)
    _expect(v, "v", lead + tail, dt)
    if fmt_bits(f) != 16:
        _expect(ks, "k_scale", lead + (D // group,), torch.float16)
        _expect(vs, "v_scale", lead + (D // group,), torch.float16)


def _validate_decode(q, k, v, ks, vs, f: Fmt, group: int, grouped: bool) -> None:
    if q.dim() != 2:
        _fail(f"q must be [H, D] (got {tuple(q.shape)})")
    H, D = q.shape
    _expect(q, "q", (H, D), torch.float16)
    _check_dg(f, D, group)
    if k.dim() != 3:
        _fail(f"k must be [heads, L, row] (got {tuple(k.shape)})")
    Hk, L = k.shape[0], k.shape[1]
    if grouped:
        _check(Hk >= 1, lambda: f"k must have at least one head (got {Hk})")
        _check(H % Hk == 0, lambda: f"query heads ({H}) must be a multiple of K/V heads ({Hk})")
    else:
        _check(Hk == H, lambda: f"k has {Hk} heads, q has {H}")
    _check_kv(f, k, v, ks, vs, (Hk, L), D, group)


def _validate_paged(q, kp, vp, ksp, vsp, block_table, seq_lens, f: Fmt, group: int) -> None:
    if q.dim() != 3:
        _fail(f"q must be [B, Hq, D] (got {tuple(q.shape)})")
    B, Hq, D = q.shape
    _expect(q, "q", (B, Hq, D), torch.float16)
    _check_dg(f, D, group)
    if kp.dim() != 4:
        _fail(f"k_pages must be [num_pages, Hkv, page_rows, row] (got {tuple(kp.shape)})")
    num_pages, Hkv, page_rows = kp.shape[:3]
    _check(Hkv >= 1, lambda: f"k_pages must have at least one head (got {Hkv})")
    _check(Hq % Hkv == 0, lambda: f"query heads ({Hq}) must be a multiple of K/V heads ({Hkv})")
    _check_kv(f, kp, vp, ksp, vsp, (num_pages, Hkv, page_rows), D, group)
    if block_table.dim() != 2:
        _fail(f"block_table must be [B={B}, max_pages] (got {tuple(block_table.shape)})")
    _check(block_table.shape[0] == B, lambda: f"block_table must be [B={B}, max_pages] (got {tuple(block_table.shape)})")
    _expect(block_table, "block_table", (B, block_table.shape[1]), torch.int32)
    _expect(seq_lens, "seq_lens", (B,), torch.int32)


def _validate_append(x, start, block_table, pages, scale_pages, f: Fmt, group: int) -> None:
    if x.dim() != 4:
        _fail(f"x must be [B, Hkv, n, D] (got {tuple(x.shape)})")
    B, Hkv, n, D = x.shape
    _expect(x, "x", (B, Hkv, n, D), torch.float16)
    _check_dg(f, D, group)
    if pages.dim() != 4:
        _fail(f"pages must be [num_pages, Hkv, page_rows, row] (got {tuple(pages.shape)})")
    num_pages, Hp, page_rows = pages.shape[:3]
    _check(Hp == Hkv, lambda: f"pages hold {Hp} K/V heads, x has {Hkv}")
    tail, dt = _row_shape(f, D)
    _expect(pages, "pages", (num_pages, Hkv, page_rows) + tail, dt)
    if fmt_bits(f) != 16:
        _expect(scale_pages, "scale_pages", (num_pages, Hkv, page_rows, D // group), torch.float16)
    _expect(start, "start", (B,), torch.int32)
    if block_table.dim() != 2:
        _fail(f"block_table must be [B={B}, max_pages] (got {tuple(block_table.shape)})")
    _check(block_table.shape[0] == B, lambda: f"block_table must be [B={B}, max_pages] (got {tuple(block_table.shape)})")
    _expect(block_table, "block_table", (B, block_table.shape[1]), torch.int32)


def _validate_quantize(x, bits: int, group: int) -> None:
    if bits not in (8, 4, 3):
        _fail(f"bits must be 8, 4 or 3 (got {bits})")
    if x.dtype != torch.float32:
        _fail(f"x must be fp32 (got {x.dtype})")
    if group not in (32, 64):
        _fail(f"group must be 32 or 64 (got {group})")
    if x.dim() == 0:
        _fail("x must have a last dimension D")
    D = x.shape[-1]
    _check((D >= group) & (D % group == 0) & (D % 8 == 0),
           lambda: f"group must be 32 or 64 and divide D (got group={group}, D={D})")


def _validate_dequantize(packed, scales, bits: int, group: int):
    """Checks packed uint8 [..., D*bits/8] and scales fp16 [..., D/G]; returns D."""
    if bits not in (8, 4, 3):
        _fail(f"bits must be 8, 4 or 3 (got {bits})")
    if packed.dtype != torch.uint8:
        _fail(f"packed must be uint8 (got {packed.dtype})")
    if group not in (32, 64):
        _fail(f"group must be 32 or 64 (got {group})")
    if packed.dim() == 0:
        _fail("packed must have a last dimension (row bytes)")
    nb = packed.shape[-1]
    _check(nb * 8 % bits == 0, lambda: f"packed rows of {nb} bytes do not hold whole {bits}-bit codes")
    D = nb * 8 // bits
    _check((D >= group) & (D % group == 0) & (D % 8 == 0),
           lambda: f"group must be 32 or 64 and divide D (got group={group}, D={D})")
    _expect(scales, "scales", tuple(packed.shape[:-1]) + (D // group,), torch.float16)
    return D


@torch.library.custom_op("voltattn::decode", mutates_args=())
def decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, k_scale: Optional[torch.Tensor],
           v_scale: Optional[torch.Tensor], fmt: str, group: int = 32, splits: int = 0) -> torch.Tensor:
    """q fp16 [H, D]; k, v [H, L, row] (uint8) or [H, L, D] (fp16 formats); scales fp16 [H, L, D/G]."""
    f = _fmt(fmt)
    _validate_decode(q, k, v, k_scale, v_scale, f, group, grouped=False)
    _need_gpu(q, k, v, k_scale, v_scale)
    H, D, L = int(q.shape[0]), _D_of(q), int(k.shape[1])
    S = splits
    if S <= 0:
        s = C.c_int(0)
        check(lib.va_pick_splits(int(f), H, L, D, C.byref(s)))
        S = s.value
    out = torch.empty((H, D), dtype=torch.float16, device=q.device)
    ws = torch.empty(ws_bytes(H, D, S) // 4, dtype=torch.float32, device=q.device)
    b = _Bufs(_ptr(k), _ptr(v), _ptr(k_scale), _ptr(v_scale), _ptr(q), _ptr(out), _ptr(ws))
    check(lib.va_decode(int(f), C.byref(b), H, L, D, group, S, _stream(q)))
    return out


@decode.register_fake
def _(q, k, v, k_scale, v_scale, fmt, group=32, splits=0):
    _validate_decode(q, k, v, k_scale, v_scale, _fmt(fmt), group, grouped=False)
    return q.new_empty((q.shape[0], q.shape[-1]), dtype=torch.float16)


@torch.library.custom_op("voltattn::decode_gqa", mutates_args=())
def decode_gqa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, k_scale: Optional[torch.Tensor],
               v_scale: Optional[torch.Tensor], fmt: str, group: int = 32, splits: int = 0) -> torch.Tensor:
    """q fp16 [Hq, D]; k, v [Hkv, L, ...]; query head h attends KV head h // (Hq / Hkv)."""
    f = _fmt(fmt)
    _validate_decode(q, k, v, k_scale, v_scale, f, group, grouped=True)
    _need_gpu(q, k, v, k_scale, v_scale)
    Hq, Hkv, D, L = int(q.shape[0]), int(k.shape[0]), _D_of(q), int(k.shape[1])
    S = splits
    if S <= 0:
        s = C.c_int(0)
        check(lib.va_pick_splits_gqa(int(f), Hq, Hkv, L, D, C.byref(s)))
        S = s.value
    out = torch.empty((Hq, D), dtype=torch.float16, device=q.device)
    ws = torch.empty(ws_bytes(Hq, D, S) // 4, dtype=torch.float32, device=q.device)
    b = _Bufs(_ptr(k), _ptr(v), _ptr(k_scale), _ptr(v_scale), _ptr(q), _ptr(out), _ptr(ws))
    check(lib.va_decode_gqa(int(f), C.byref(b), Hq, Hkv, L, D, group, S, _stream(q)))
    return out


@decode_gqa.register_fake
def _(q, k, v, k_scale, v_scale, fmt, group=32, splits=0):
    _validate_decode(q, k, v, k_scale, v_scale, _fmt(fmt), group, grouped=True)
    return q.new_empty((q.shape[0], q.shape[-1]), dtype=torch.float16)


def _paged_shape(q, k_pages, block_table, group, max_seq_len):
    B, Hq, D = (int(x) for x in q.shape)
    num_pages, Hkv, page_rows = (int(x) for x in k_pages.shape[:3])
    return _PagedShape(B, Hq, Hkv, D, group, page_rows, int(block_table.shape[1]), num_pages,
                       max_seq_len)


@torch.library.custom_op("voltattn::decode_paged", mutates_args=())
def decode_paged(q: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor,
                 k_scale_pages: Optional[torch.Tensor], v_scale_pages: Optional[torch.Tensor],
                 block_table: torch.Tensor, seq_lens: torch.Tensor, fmt: str, max_seq_len: int,
                 group: int = 32, splits: int = 0) -> torch.Tensor:
    """q fp16 [B, Hq, D]; pages [num_pages, Hkv, page_rows, ...]; block_table int32
    [B, max_pages]; seq_lens int32 [B] (each <= max_seq_len)."""
    f = _fmt(fmt)
    _validate_paged(q, k_pages, v_pages, k_scale_pages, v_scale_pages, block_table, seq_lens, f, group)
    _need_gpu(q, k_pages, v_pages, k_scale_pages, v_scale_pages, block_table, seq_lens)
    shape = _paged_shape(q, k_pages, block_table, group, max_seq_len)
    S = splits
    if S <= 0:
        s = C.c_int(0)
        check(lib.va_pick_splits_paged(int(f), C.byref(shape), C.byref(s)))
        S = s.value
    B, Hq, D = (int(x) for x in q.shape)
    out = torch.empty((B, Hq, D), dtype=torch.float16, device=q.device)
    ws = torch.empty(ws_bytes(B * Hq, D, S) // 4, dtype=torch.float32, device=q.device)
    b = _PagedBufs(_ptr(k_pages), _ptr(v_pages), _ptr(k_scale_pages), _ptr(v_scale_pages),
                   _ptr(block_table), _ptr(seq_lens), _ptr(q), _ptr(out), _ptr(ws))
    check(lib.va_decode_paged(int(f), C.byref(b), C.byref(shape), S, _stream(q)))
    return out


@decode_paged.register_fake
def _(q, k_pages, v_pages, k_scale_pages, v_scale_pages, block_table, seq_lens, fmt, max_seq_len,
      group=32, splits=0):
    _validate_paged(q, k_pages, v_pages, k_scale_pages, v_scale_pages, block_table, seq_lens, _fmt(fmt), group)
    return q.new_empty(q.shape, dtype=torch.float16)


@torch.library.custom_op("voltattn::append_kv", mutates_args=("pages", "scale_pages"))
def append_kv(x: torch.Tensor, start: torch.Tensor, block_table: torch.Tensor, pages: torch.Tensor,
              scale_pages: Optional[torch.Tensor], fmt: str, group: int = 32) -> None:
    """x fp16 [B, Hkv, n, D] new rows written at positions start[b] + r of the paged cache
    pages [num_pages, Hkv, page_rows, ...] (+ scale_pages for quantized formats)."""
    f = _fmt(fmt)
    _validate_append(x, start, block_table, pages, scale_pages, f, group)
    _need_gpu(x, start, block_table, pages, scale_pages)
    B, Hkv, n, D = (int(s) for s in x.shape)
    num_pages, _, page_rows = (int(s) for s in pages.shape[:3])
    shape = _PagedShape(B, Hkv, Hkv, D, group, page_rows, int(block_table.shape[1]), num_pages, 0)
    check(lib.va_append_kv(int(f), _ptr(x), n, _ptr(start), _ptr(block_table), C.byref(shape),
                           _ptr(pages), _ptr(scale_pages), _stream(x)))


@append_kv.register_fake
def _(x, start, block_table, pages, scale_pages, fmt, group=32):
    _validate_append(x, start, block_table, pages, scale_pages, _fmt(fmt), group)
    return None


@torch.library.custom_op("voltattn::quantize", mutates_args=())
def quantize(x: torch.Tensor, bits: int, group: int = 32) -> tuple[torch.Tensor, torch.Tensor]:
    """x fp32 [..., D] -> (packed uint8 [..., D*bits/8], fp16 scales [..., D/G])."""
    _validate_quantize(x, bits, group)
    _need_gpu(x)
    D = int(x.shape[-1])
    rows = x.numel() // D
    packed = torch.empty(x.shape[:-1] + (D * bits // 8,), dtype=torch.uint8, device=x.device)
    scales = torch.empty(x.shape[:-1] + (D // group,), dtype=torch.float16, device=x.device)
    check(lib.va_quantize(bits, group, _ptr(x), rows, D, _ptr(packed), _ptr(scales), _stream(x)))
    return packed, scales


@quantize.register_fake
def _(x, bits, group=32):
    _validate_quantize(x, bits, group)
    D = x.shape[-1]
    return (x.new_empty(x.shape[:-1] + (D * bits // 8,), dtype=torch.uint8),
            x.new_empty(x.shape[:-1] + (D // group,), dtype=torch.float16))


@torch.library.custom_op("voltattn::dequantize", mutates_args=())
def dequantize(packed: torch.Tensor, scales: torch.Tensor, bits: int, group: int = 32) -> torch.Tensor:
    """(packed uint8 [..., D*bits/8], fp16 scales [..., D/G]) -> fp32 [..., D], bit-exact dq()."""
    D = int(_validate_dequantize(packed, scales, bits, group))
    _need_gpu(packed, scales)
    rows = packed.numel() // max(1, int(packed.shape[-1]))
    out = torch.empty(packed.shape[:-1] + (D,), dtype=torch.float32, device=packed.device)
    check(lib.va_dequantize(bits, group, _ptr(packed), _ptr(scales), rows, D, _ptr(out), _stream(packed)))
    return out


@dequantize.register_fake
def _(packed, scales, bits, group=32):
    D = _validate_dequantize(packed, scales, bits, group)
    return packed.new_empty(packed.shape[:-1] + (D,), dtype=torch.float32)


def row_format_bits(fmt: str) -> int:
    return fmt_bits(_fmt(fmt))
