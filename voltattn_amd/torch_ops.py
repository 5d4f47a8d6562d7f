"""PyTorch-ROCm binding: ``torch.ops.voltattn.*`` custom ops over the C ABI.

Importing this module registers

* ``voltattn::decode(q, k, v, k_scale, v_scale, fmt, group, splits) -> out``
  — one decode step (va_decode; the reference's launch(), src/voltattn.cu:803-835);
* ``voltattn::decode_gqa(...)`` — Hq query heads over Hkv KV heads (va_decode_gqa);
* ``voltattn::decode_paged(...)`` — a batch over a page pool (va_decode_paged);
* ``voltattn::append_kv(...)`` — quantize-and-append new rows (va_append_kv; mutates the pools);
* ``voltattn::quantize(x, bits, group) -> (packed, scales)`` (va_quantize; the reference's
  quantize(), src/voltattn.cu:705-745).

Tensors keep the C ABI's layouts (include/voltattn.h): q/out fp16 [.., H, D];
quantized K/V payload uint8 [.., L, row bytes]; f16 K/V fp16 [.., L, D]; scales
fp16 [.., L, D/G]. Every op runs asynchronously on torch's current HIP stream
and fails loudly (RuntimeError with the library's message) on invalid input;
there is no CPU fallback: the tensors must live on a gfx950 device. Each op has
a fake (meta) implementation, so shapes propagate under torch.compile.
"""
from __future__ import annotations

import ctypes as C
from typing import Optional

import torch

from . import (Fmt, _Bufs, _PagedBufs, _PagedShape, check, fmt_bits, lib, ws_bytes)

__all__ = ["decode", "decode_gqa", "decode_paged", "append_kv", "quantize"]


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


@torch.library.custom_op("voltattn::decode", mutates_args=())
def decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, k_scale: Optional[torch.Tensor],
           v_scale: Optional[torch.Tensor], fmt: str, group: int = 32, splits: int = 0) -> torch.Tensor:
    """q fp16 [H, D]; k, v [H, L, row] (uint8) or [H, L, D] (fp16 formats); scales fp16 [H, L, D/G]."""
    _need_gpu(q, k, v, k_scale, v_scale)
    f = _fmt(fmt)
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
    return q.new_empty((q.shape[0], q.shape[-1]), dtype=torch.float16)


@torch.library.custom_op("voltattn::decode_gqa", mutates_args=())
def decode_gqa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, k_scale: Optional[torch.Tensor],
               v_scale: Optional[torch.Tensor], fmt: str, group: int = 32, splits: int = 0) -> torch.Tensor:
    """q fp16 [Hq, D]; k, v [Hkv, L, ...]; query head h attends KV head h // (Hq / Hkv)."""
    _need_gpu(q, k, v, k_scale, v_scale)
    f = _fmt(fmt)
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
    _need_gpu(q, k_pages, v_pages, k_scale_pages, v_scale_pages, block_table, seq_lens)
    if block_table.dtype != torch.int32 or seq_lens.dtype != torch.int32:
        raise RuntimeError("block_table and seq_lens must be int32")
    f = _fmt(fmt)
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
    return q.new_empty(q.shape, dtype=torch.float16)


@torch.library.custom_op("voltattn::append_kv", mutates_args=("pages", "scale_pages"))
def append_kv(x: torch.Tensor, start: torch.Tensor, block_table: torch.Tensor, pages: torch.Tensor,
              scale_pages: Optional[torch.Tensor], fmt: str, group: int = 32) -> None:
    """x fp16 [B, Hkv, n, D] new rows written at positions start[b] + r of the paged cache
    pages [num_pages, Hkv, page_rows, ...] (+ scale_pages for quantized formats)."""
    _need_gpu(x, start, block_table, pages, scale_pages)
    if x.dtype != torch.float16:
        raise RuntimeError("x must be fp16")
    f = _fmt(fmt)
    B, Hkv, n, D = (int(s) for s in x.shape)
    num_pages, _, page_rows = (int(s) for s in pages.shape[:3])
    shape = _PagedShape(B, Hkv, Hkv, D, group, page_rows, int(block_table.shape[1]), num_pages, 0)
    check(lib.va_append_kv(int(f), _ptr(x), n, _ptr(start), _ptr(block_table), C.byref(shape),
                           _ptr(pages), _ptr(scale_pages), _stream(x)))


@append_kv.register_fake
def _(x, start, block_table, pages, scale_pages, fmt, group=32):
    return None


@torch.library.custom_op("voltattn::quantize", mutates_args=())
def quantize(x: torch.Tensor, bits: int, group: int = 32) -> tuple[torch.Tensor, torch.Tensor]:
    """x fp32 [..., D] -> (packed uint8 [..., D*bits/8], fp16 scales [..., D/G])."""
    _need_gpu(x)
    if x.dtype != torch.float32:
        raise RuntimeError("x must be fp32")
    D = int(x.shape[-1])
    rows = x.numel() // D
    packed = torch.empty(x.shape[:-1] + (D * bits // 8,), dtype=torch.uint8, device=x.device)
    scales = torch.empty(x.shape[:-1] + (D // group,), dtype=torch.float16, device=x.device)
    check(lib.va_quantize(bits, group, _ptr(x), rows, D, _ptr(packed), _ptr(scales), _stream(x)))
    return packed, scales


@quantize.register_fake
def _(x, bits, group=32):
    D = x.shape[-1]
    return (x.new_empty(x.shape[:-1] + (D * bits // 8,), dtype=torch.uint8),
            x.new_empty(x.shape[:-1] + (D // group,), dtype=torch.float16))


def row_format_bits(fmt: str) -> int:
    return fmt_bits(_fmt(fmt))
