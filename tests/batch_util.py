"""Host-side builders of grouped-query and paged decode cases for the GPU tests.

K/V rows come from the oracle's seeded draws and quantizer (oracle.make_case:
the reference's run_case inputs, src/voltattn.cu:838-861); query heads are
seeded fp16 N(0,1) draws; the expected output is the oracle's double
reference over the dequantized rows (oracle.batch.reference_gqa)."""
from __future__ import annotations

import numpy as np

import oracle
from oracle import batch
import voltattn_amd as va


def f16(x) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def kv_case(fmt: va.Fmt, Hkv: int, L: int, D: int, G: int, seed: int) -> dict:
    """Quantized (or fp16) K/V of Hkv heads x L rows, as [Hkv][L][row bytes] arrays."""
    bits = va.fmt_bits(fmt)
    c = oracle.make_case(bits, Hkv, L, D, G, seed)
    rb = va.row_bytes(fmt, D)
    out = {
        "kpay": c["kpay"].reshape(Hkv, L, rb), "vpay": c["vpay"].reshape(Hkv, L, rb),
        "kd": c["kd"], "vd": c["vd"], "ksc": None, "vsc": None,
    }
    if bits != 16:
        out["ksc"] = c["ksc"].reshape(Hkv, L, D // G)
        out["vsc"] = c["vsc"].reshape(Hkv, L, D // G)
    return out


def queries(n_heads: int, D: int, seed: int) -> np.ndarray:
    return f16(np.random.default_rng(seed).standard_normal(n_heads * D)).reshape(n_heads, D)


class PagedBatch:
    """A batch of sequences in a page pool, uploaded to the device."""

    def __init__(self, fmt: va.Fmt, lens, Hq: int, Hkv: int, D: int, G: int, page_rows: int,
                 seed: int, extra_pages: int = 3, max_seq_len: int | None = None,
                 max_pages: int | None = None):
        self.fmt, self.lens, self.Hq, self.Hkv, self.D, self.G = fmt, list(lens), Hq, Hkv, D, G
        self.P = page_rows
        B = len(self.lens)
        rng = np.random.default_rng(seed)
        need = [-(-L // page_rows) for L in self.lens]
        self.max_pages = max_pages or max(1, max(need))
        num_pages = sum(need) + extra_pages
        perm = rng.permutation(num_pages)
        self.table = np.full((B, self.max_pages), -7, np.int32)   # unused entries: invalid ids
        at = 0
        for b, n in enumerate(need):
            self.table[b, :n] = perm[at:at + n]
            at += n
        rb = va.row_bytes(fmt, D)
        quant = va.fmt_bits(fmt) != 16
        # garbage everywhere the batch does not write (fp16 NaN/Inf patterns included)
        self.kpool = rng.integers(0, 256, (num_pages, Hkv, page_rows, rb), dtype=np.uint8)
        self.vpool = rng.integers(0, 256, (num_pages, Hkv, page_rows, rb), dtype=np.uint8)
        self.kspool = self.vspool = None
        if quant:
            self.kspool = rng.integers(0, 65536, (num_pages, Hkv, page_rows, D // G), dtype=np.uint16)
            self.vspool = rng.integers(0, 65536, (num_pages, Hkv, page_rows, D // G), dtype=np.uint16)
        self.q = queries(B * Hq, D, seed + 1).reshape(B, Hq, D)
        self.ref = np.zeros((B, Hq, D), np.float32)
        self.mag = np.zeros((B, Hq, D), np.float64)     # sum_j p_j |v_jd| (error scale of cancelling outputs)
        for b, L in enumerate(self.lens):
            if L == 0:
                continue
            c = kv_case(fmt, Hkv, L, D, G, seed * 7919 + b)
            batch.scatter_rows(self.kpool, c["kpay"], self.table[b], page_rows)
            batch.scatter_rows(self.vpool, c["vpay"], self.table[b], page_rows)
            if quant:
                batch.scatter_rows(self.kspool, c["ksc"], self.table[b], page_rows)
                batch.scatter_rows(self.vspool, c["vsc"], self.table[b], page_rows)
            self.ref[b] = batch.reference_gqa(c["kd"], c["vd"], self.q[b], Hq, Hkv, L, D).reshape(Hq, D)
            self.mag[b] = batch.magnitude_gqa(c["kd"], c["vd"], self.q[b], Hq, Hkv, L, D).reshape(Hq, D)
        self.shape = va.PagedShape(B, Hq, Hkv, D, G, page_rows, self.max_pages, num_pages,
                                   max_seq_len if max_seq_len is not None else max(max(self.lens), 1))
        self.seq_lens = np.asarray(self.lens, np.int32)
        self.bufs = []

    def _dev(self, a):
        d = va.DeviceBuffer.from_array(a)
        self.bufs.append(d)
        return d.ptr

    def run(self, S: int = 0, seq_lens=None, table=None) -> np.ndarray:
        B = len(self.lens)
        quant = self.kspool is not None
        Sx = S or va.pick_splits_paged(self.fmt, self.shape)
        out = va.DeviceBuffer(B * self.Hq * self.D * 2)
        ws = va.DeviceBuffer(va.ws_bytes(B * self.Hq, self.D, Sx))
        self.bufs += [out, ws]
        b = va.PagedBufs(
            K=self._dev(self.kpool), V=self._dev(self.vpool),
            scK=self._dev(self.kspool) if quant else 0, scV=self._dev(self.vspool) if quant else 0,
            block_table=self._dev(self.table if table is None else table),
            seq_lens=self._dev(self.seq_lens if seq_lens is None else np.asarray(seq_lens, np.int32)),
            q=self._dev(self.q), out=out.ptr, ws=ws.ptr)
        va.decode_paged(self.fmt, b, self.shape, S)
        va.sync()
        return out.download(np.uint16).view(np.float16).astype(np.float32).reshape(B, self.Hq, self.D)

    def free(self):
        for d in self.bufs:
            d.free()
        self.bufs = []


def kv_from_values(fmt: va.Fmt, xk: np.ndarray, xv: np.ndarray, G: int) -> dict:
    """K/V of chosen fp32 values [Hkv][L][D]: the reference's quantizer (quantize(),
    src/voltattn.cu:705-745) for the quantized formats, fp16 rounding for f16."""
    Hkv, L, D = xk.shape
    bits = va.fmt_bits(fmt)
    rb = va.row_bytes(fmt, D)
    out = {"ksc": None, "vsc": None}
    for name, x in (("k", xk), ("v", xv)):
        x = np.ascontiguousarray(x, np.float32)
        if bits == 16:
            h = x.astype(np.float16)
            out[name + "pay"] = h.view(np.uint8).reshape(Hkv, L, rb)
            out[name + "d"] = h.astype(np.float32).ravel()
        else:
            data, scale = oracle.quantize(x, D, G, bits)
            out[name + "pay"] = data.reshape(Hkv, L, rb)
            out[name + "sc"] = scale.reshape(Hkv, L, D // G)
            out[name + "d"] = oracle.dequant(data, scale, Hkv * L, D, G, bits)
    return out
