"""GPU parity of grouped-query decode on inputs far from N(0, 1): magnitudes that
stress the fp32 and fp16 ranges the kernels work in (the matrix-core form's
power-of-two row exponents, fp16 hi + lo weights and exact q digits; the VALU
form's lazy running maximum). Each case is built on the host, quantized with the
reference's quantizer (src/voltattn.cu:705-745) and checked against the oracle's
double reference (oracle.batch.reference_gqa) with the reference's gate
(src/voltattn.cu:903) and the tight bound (half an fp16 ulp + 2e-6 relative),
widened by the error any fp32 kernel makes on these inputs: a score is an fp32
dot whose rounding is a few ulps of sum_d |q_d k_d| (in log2 units), which
moves each weight by that much relatively and the output by that times max|v|
(negligible for N(0, 1)-like data; large when |q.k| terms are huge and cancel)."""
import zlib

import numpy as np
import pytest

import oracle
from oracle import batch
import voltattn_amd as va
from tests import batch_util
from tests.numerics import tight_bound

pytestmark = pytest.mark.gpu

TILED = [va.Fmt.F16M, va.Fmt.Q8M, va.Fmt.Q4M, va.Fmt.Q3M]
L, D, G = 3000, 128, 32


def _values(kind: str, rng, Hq: int, Hkv: int):
    xk = rng.standard_normal((Hkv, L, D)).astype(np.float32)
    xv = rng.standard_normal((Hkv, L, D)).astype(np.float32)
    q = rng.standard_normal((Hq, D)).astype(np.float32)
    if kind == "row_scales":          # per-position magnitudes from 1e-4 to 1e3
        xk *= (10.0 ** rng.uniform(-4, 3, (Hkv, L, 1))).astype(np.float32)
        xv *= (10.0 ** rng.uniform(-4, 3, (Hkv, L, 1))).astype(np.float32)
        q *= 0.01
    elif kind == "group_scales":      # each scale group of a row on its own scale
        f = (10.0 ** rng.uniform(-3, 3, (Hkv, L, D // G, 1))).astype(np.float32)
        xk = (xk.reshape(Hkv, L, D // G, G) * f).reshape(Hkv, L, D)
        f = (10.0 ** rng.uniform(-3, 3, (Hkv, L, D // G, 1))).astype(np.float32)
        xv = (xv.reshape(Hkv, L, D // G, G) * f).reshape(Hkv, L, D)
        q *= 0.05
    elif kind == "sharp":             # large q: one position dominates, many new maxima
        q *= 60.0
    elif kind == "flat":              # tiny q: nearly uniform weights over 3000 positions
        q *= 1e-3
    elif kind == "rising":            # scores grow along L: the running maximum keeps moving
        u = np.sign(q[0]).astype(np.float32)
        xk += np.linspace(0, 0.3, L, dtype=np.float32)[None, :, None] * u[None, None, :]
    elif kind == "zero_groups":       # all-zero groups (scale 1) and groups whose scale underflows to 0
        xk[:, ::7, :G] = 0.0
        xv[:, ::5, G:2 * G] = 0.0
        xv[:, 1::5, 2 * G:3 * G] *= 1e-9
        xk[:, 2::11, 3 * G:] *= 1e-9
    elif kind == "big_v":             # V near the fp16 range: operand exponents must scale down
        xv *= 2000.0
    return xk, xv, q


@pytest.mark.parametrize("fmt", TILED, ids=lambda f: f.label)
@pytest.mark.parametrize("kind", ["row_scales", "group_scales", "sharp", "flat", "rising",
                                  "zero_groups", "big_v"])
@pytest.mark.parametrize("heads", [(8, 2), (4, 4)], ids=lambda h: f"Hq{h[0]}-Hkv{h[1]}")
def test_gqa_value_ranges(fmt, kind, heads):
    """Hq = Hkv is the reference shape (va_decode_gqa forwards it to va_decode)."""
    Hq, Hkv = heads
    rng = np.random.default_rng(zlib.crc32(f"{kind}/{fmt.label}/{Hq}".encode()))
    xk, xv, q = _values(kind, rng, Hq, Hkv)
    c = batch_util.kv_from_values(fmt, xk, xv, G)
    qh = batch_util.f16(q.ravel()).reshape(Hq, D)
    print(f"gqa range {fmt.label} {kind} Hq={Hq} Hkv={Hkv}", flush=True)
    bufs = []
    try:
        dev = lambda a: bufs.append(va.DeviceBuffer.from_array(a)) or bufs[-1].ptr
        S = va.pick_splits_gqa(fmt, Hq, Hkv, L, D)
        out = va.DeviceBuffer(Hq * D * 2)
        ws = va.DeviceBuffer(va.ws_bytes(Hq, D, S))
        bufs += [out, ws]
        b = va.DeviceBufs(K=dev(c["kpay"]), V=dev(c["vpay"]),
                          scK=dev(c["ksc"]) if c["ksc"] is not None else 0,
                          scV=dev(c["vsc"]) if c["vsc"] is not None else 0,
                          q=dev(qh), out=out.ptr, ws=ws.ptr)
        va.decode_gqa(fmt, b, Hq, Hkv, L, D, S=S, G=G)
        va.sync()
        got = out.download(np.uint16).view(np.float16).astype(np.float32)
    finally:
        for x in bufs:
            x.free()
    ref = batch.reference_gqa(c["kd"], c["vd"], qh, Hq, Hkv, L, D)
    assert np.all(np.isfinite(ref)), kind
    assert np.all(np.isfinite(got)), (fmt.label, kind)
    ok, maxerr = oracle.gate(got, ref)
    assert ok, (fmt.label, kind, maxerr)
    tb = tight_bound(ref)
    print(f"  err/tight max {float((np.abs(got - ref) / tb).max()):.3g}", flush=True)
    bound = tb + _fp32_score_term(c, qh, Hq, Hkv).ravel()
    bad = np.abs(got - ref) > bound
    assert not bad.any(), (fmt.label, kind, int(bad.sum()), float(np.abs(got - ref).max()),
                           float((np.abs(got - ref) / bound).max()))


def _fp32_score_term(c, qh, Hq, Hkv):
    """Per query head: 2 * max|v| * 8 ulp(fp32) * ln2 * max_j sum_d |q_d k_jd| * log2(e)/sqrt(D)."""
    kd = c["kd"].reshape(Hkv, L, D).astype(np.float64)
    vd = c["vd"].reshape(Hkv, L, D).astype(np.float64)
    q = qh.view(np.float16).astype(np.float64).reshape(Hq, D)
    g = Hq // Hkv
    term = np.empty((Hq, D))
    for h in range(Hq):
        cond = (np.abs(kd[h // g]) @ np.abs(q[h])).max() * np.log2(np.e) / np.sqrt(D)
        eps = 8 * 2.0 ** -24 * cond * np.log(2)
        term[h] = 2 * np.abs(vd[h // g]).max() * eps
    return term
