"""GPU parity of the torch.library ops (torch.ops.voltattn.*) against a plain
PyTorch fp32 reference: softmax(q.K^T / sqrt(D)).V over the K/V values the
oracle's dequant gives for the packed bytes (dq(), src/voltattn.cu:747-767).
Tolerance: the tight bound of tests/numerics.py (half an fp16 ulp + 2e-6|ref|)
plus 2e-6 absolute for the fp32 reference's own rounding. quantize and
append_kv are checked bit for bit against the oracle's quantizer, dequantize
against the oracle's dq()."""
import numpy as np
import pytest
import torch

import oracle
import voltattn_amd as va
import voltattn_amd.torch_ops  # noqa: F401
from tests.numerics import tight_bound

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _ref(q, kd, vd, Hq, Hkv):
    """fp32 torch attention; kd, vd [Hkv, L, D] fp32, q [Hq, D] fp16."""
    g = Hq // Hkv
    k = torch.as_tensor(kd).float().repeat_interleave(g, 0)
    v = torch.as_tensor(vd).float().repeat_interleave(g, 0)
    qf = q.float().cpu()
    s = torch.einsum("hd,hld->hl", qf, k) / np.sqrt(q.shape[-1])
    return torch.einsum("hl,hld->hd", torch.softmax(s, -1), v)


def _kv(fmt, H, L, D, G, seed):
    """(payload, scales, dequantized fp32) of K or V through the op-level quantizer."""
    x = torch.randn(H, L, D, generator=torch.Generator().manual_seed(seed))
    bits = va.fmt_bits(va.Fmt.parse(fmt))
    if bits == 16:
        h = x.half()
        return h.to(DEV), None, h.float().numpy()
    packed, scales = torch.ops.voltattn.quantize(x.to(DEV), bits, G)
    torch.cuda.synchronize()
    p, s = packed.cpu().numpy(), scales.cpu().numpy().view(np.uint16)
    deq = oracle.dequant(p.ravel(), s.ravel(), H * L, D, G, bits).reshape(H, L, D)
    return packed, scales, deq


def _close(got, ref):
    got = got.float().cpu().numpy()
    ref = ref.numpy()
    assert np.all(np.isfinite(got))
    err = np.abs(got - ref)
    assert np.all(err <= tight_bound(ref) + 2e-6), float(err.max())


@pytest.mark.parametrize("fmt", ["f16+", "q8+", "q4+", "q3+", "q8"])
def test_decode_op(fmt):
    H, L, D, G = 8, 1000, 128, 32
    k, ks, kd = _kv(fmt, H, L, D, G, 1)
    v, vs, vd = _kv(fmt, H, L, D, G, 2)
    q = torch.randn(H, D, generator=torch.Generator().manual_seed(3)).half().to(DEV)
    out = torch.ops.voltattn.decode(q, k, v, ks, vs, fmt, G)
    _close(out, _ref(q, kd, vd, H, H))


@pytest.mark.parametrize("fmt", ["f16+", "q8+", "q4+", "q3+"])
def test_decode_gqa_op(fmt):
    Hq, Hkv, L, D, G = 16, 4, 777, 128, 32
    k, ks, kd = _kv(fmt, Hkv, L, D, G, 4)
    v, vs, vd = _kv(fmt, Hkv, L, D, G, 5)
    q = torch.randn(Hq, D, generator=torch.Generator().manual_seed(6)).half().to(DEV)
    out = torch.ops.voltattn.decode_gqa(q, k, v, ks, vs, fmt, G)
    _close(out, _ref(q, kd, vd, Hq, Hkv))


@pytest.mark.parametrize("fmt", ["f16+", "q8+", "q4+"])
def test_append_then_decode_paged_ops(fmt):
    """A serving step: append rows into a paged cache with the op, decode with the op."""
    B, Hq, Hkv, D, G, P, npg = 3, 8, 2, 128, 32, 64, 4
    lens = [200, 64, 1]
    bits = va.fmt_bits(va.Fmt.parse(fmt))
    rb = D * bits // 8
    gen = torch.Generator().manual_seed(7)
    num_pages = B * npg
    table = torch.randperm(num_pages, generator=gen).int().reshape(B, npg)
    if bits == 16:
        kp = torch.zeros(num_pages, Hkv, P, D, dtype=torch.float16, device=DEV)
        kps = None
    else:
        kp = torch.zeros(num_pages, Hkv, P, rb, dtype=torch.uint8, device=DEV)
        kps = torch.zeros(num_pages, Hkv, P, D // G, dtype=torch.float16, device=DEV)
    vp = torch.zeros_like(kp)
    vps = None if kps is None else torch.zeros_like(kps)
    xk = torch.randn(B, Hkv, max(lens), D, generator=gen).half()
    xv = torch.randn(B, Hkv, max(lens), D, generator=gen).half()
    bt = table.to(DEV)
    zero = torch.zeros(B, dtype=torch.int32, device=DEV)
    torch.ops.voltattn.append_kv(xk.to(DEV), zero, bt, kp, kps, fmt, G)
    torch.ops.voltattn.append_kv(xv.to(DEV), zero, bt, vp, vps, fmt, G)
    q = torch.randn(B, Hq, D, generator=gen).half().to(DEV)
    sl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    out = torch.ops.voltattn.decode_paged(q, kp, vp, kps, vps, bt, sl, fmt, max(lens), G)
    for b, L in enumerate(lens):
        deq = []
        for x in (xk, xv):
            rows = x[b, :, :L].float().numpy().reshape(-1)
            if bits == 16:
                deq.append(rows.reshape(Hkv, L, D))
            else:
                data, sc = oracle.quantize(rows, D, G, bits)
                deq.append(oracle.dequant(data, sc, Hkv * L, D, G, bits).reshape(Hkv, L, D))
        _close(out[b], _ref(q[b], deq[0], deq[1], Hq, Hkv))


@pytest.mark.parametrize("bits", [8, 4, 3])
def test_quantize_op_is_bit_exact(bits):
    x = torch.randn(64, 128, generator=torch.Generator().manual_seed(bits))
    packed, scales = torch.ops.voltattn.quantize(x.to(DEV), bits, 32)
    data, sc = oracle.quantize(x.numpy().ravel(), 128, 32, bits)
    np.testing.assert_array_equal(packed.cpu().numpy().ravel(), data)
    np.testing.assert_array_equal(scales.cpu().numpy().view(np.uint16).ravel(), sc)


@pytest.mark.parametrize("bits,G", [(8, 32), (4, 64), (3, 32)])
def test_dequantize_op_is_bit_exact(bits, G):
    x = torch.randn(3, 50, 128, generator=torch.Generator().manual_seed(10 + bits))
    packed, scales = torch.ops.voltattn.quantize(x.to(DEV), bits, G)
    out = torch.ops.voltattn.dequantize(packed, scales, bits, G)
    assert out.shape == (3, 50, 128) and out.dtype == torch.float32
    want = oracle.dequant(packed.cpu().numpy().ravel(), scales.cpu().numpy().view(np.uint16).ravel(),
                          150, 128, G, bits)
    np.testing.assert_array_equal(out.cpu().numpy().ravel().view(np.uint32), want.view(np.uint32))
