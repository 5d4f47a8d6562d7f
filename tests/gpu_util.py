"""Helpers for the GPU tests: run one oracle-built case through the C ABI."""
from __future__ import annotations

import functools

import numpy as np

import oracle
import voltattn_amd as va
from tests.numerics import half_ulp, tight_bound  # noqa: F401 (re-exported)


@functools.lru_cache(maxsize=64)
def case(bits: int, H: int, L: int, D: int, G: int, seed: int) -> dict:
    return oracle.make_case(bits, H, L, D, G, seed)


def run_case(fmt: va.Fmt, c: dict, S: int, splits_only: bool = False) -> dict:
    """Upload case `c`, run one decode step with S splits, return out (and ws)."""
    H, L, D, G = c["H"], c["L"], c["D"], c["G"]
    bufs = []
    try:
        k = va.DeviceBuffer.from_array(c["kpay"]); bufs.append(k)
        v = va.DeviceBuffer.from_array(c["vpay"]); bufs.append(v)
        q = va.DeviceBuffer.from_array(c["q"]); bufs.append(q)
        sk = sv = None
        if c["ksc"] is not None:
            sk = va.DeviceBuffer.from_array(c["ksc"]); bufs.append(sk)
            sv = va.DeviceBuffer.from_array(c["vsc"]); bufs.append(sv)
        out = va.DeviceBuffer(H * D * 2); bufs.append(out)
        ws = va.DeviceBuffer(va.ws_bytes(H, D, S)); bufs.append(ws)
        b = va.DeviceBufs(K=k.ptr, V=v.ptr, scK=sk.ptr if sk else 0, scV=sv.ptr if sv else 0,
                          q=q.ptr, out=out.ptr, ws=ws.ptr)
        if splits_only:
            va.decode_splits(fmt, b, H, L, D, S, G=G)
        else:
            va.launch(fmt, b, H, L, D, S, G=G)
        va.sync()
        res = {"ws": ws.download(np.float32).reshape(H, S, D + 2)}
        if not splits_only:
            res["out"] = out.download(np.uint16).view(np.float16).astype(np.float32)
        return res
    finally:
        for x in bufs:
            x.free()
