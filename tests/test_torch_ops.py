"""The torch.library binding without a GPU: the ops are registered under
torch.ops.voltattn, their fake (meta) implementations give the documented
output shapes and reject every tensor whose shape or dtype does not match
(fmt, D, G), and CPU tensors are refused loudly (no CPU fallback)."""
import pytest
import torch

import voltattn_amd.torch_ops  # noqa: F401  (registers torch.ops.voltattn.*)


def test_ops_registered():
    for name in ("decode", "decode_gqa", "decode_paged", "append_kv", "quantize", "dequantize"):
        assert hasattr(torch.ops.voltattn, name), name


def test_fake_shapes_on_meta():
    m = dict(device="meta")
    q = torch.empty(32, 128, dtype=torch.float16, **m)
    k = torch.empty(8, 4096, 128, dtype=torch.uint8, **m)
    s = torch.empty(8, 4096, 4, dtype=torch.float16, **m)
    assert torch.ops.voltattn.decode_gqa(q, k, k, s, s, "q8+").shape == (32, 128)
    k32 = torch.empty(32, 4096, 128, dtype=torch.uint8, **m)
    s32 = torch.empty(32, 4096, 4, dtype=torch.float16, **m)
    assert torch.ops.voltattn.decode(q, k32, k32, s32, s32, "q8+").shape == (32, 128)
    qb = torch.empty(4, 32, 128, dtype=torch.float16, **m)
    pages = torch.empty(64, 8, 256, 64, dtype=torch.uint8, **m)
    sp = torch.empty(64, 8, 256, 4, dtype=torch.float16, **m)
    bt = torch.empty(4, 16, dtype=torch.int32, **m)
    sl = torch.empty(4, dtype=torch.int32, **m)
    out = torch.ops.voltattn.decode_paged(qb, pages, pages, sp, sp, bt, sl, "q4+", 4096)
    assert out.shape == (4, 32, 128) and out.dtype == torch.float16
    packed, scales = torch.ops.voltattn.quantize(torch.empty(10, 128, **m), 3, 32)
    assert packed.shape == (10, 48) and scales.shape == (10, 4)
    x = torch.ops.voltattn.dequantize(packed, scales, 3, 32)
    assert x.shape == (10, 128) and x.dtype == torch.float32
    x = torch.ops.voltattn.dequantize(torch.empty(2, 5, 32, dtype=torch.uint8, **m),
                                      torch.empty(2, 5, 1, dtype=torch.float16, **m), 4, 64)
    assert x.shape == (2, 5, 64)


def test_cpu_tensors_refused():
    q = torch.zeros(4, 128, dtype=torch.float16)
    k = torch.zeros(4, 64, 128, dtype=torch.uint8)
    s = torch.zeros(4, 64, 4, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="gfx950"):
        torch.ops.voltattn.decode(q, k, k, s, s, "q8+")
    with pytest.raises(RuntimeError, match="gfx950"):
        torch.ops.voltattn.quantize(torch.zeros(2, 128), 8, 32)
    with pytest.raises(RuntimeError, match="gfx950"):
        torch.ops.voltattn.dequantize(torch.zeros(2, 128, dtype=torch.uint8),
                                      torch.zeros(2, 4, dtype=torch.float16), 8, 32)


M = dict(device="meta")


def _t(*shape, dtype=torch.uint8):
    return torch.empty(*shape, dtype=dtype, **M)


def _decode_args(**over):
    a = dict(q=_t(8, 128, dtype=torch.float16), k=_t(8, 256, 64), v=_t(8, 256, 64),
             ks=_t(8, 256, 4, dtype=torch.float16), vs=_t(8, 256, 4, dtype=torch.float16))
    a.update(over)
    return a


@pytest.mark.parametrize("over,msg", [
    (dict(q=_t(8, 128, dtype=torch.float32)), "q has dtype"),
    (dict(q=_t(8, 96, dtype=torch.float16)), "D must be 64 or 128"),
    (dict(k=_t(8, 256, 128)), "k has shape"),                      # q8 row bytes, not q4
    (dict(v=_t(8, 255, 64)), "v has shape"),
    (dict(k=_t(4, 256, 64), v=_t(4, 256, 64)), "k has 4 heads"),
    (dict(ks=_t(8, 256, 2, dtype=torch.float16)), "k_scale has shape"),
    (dict(vs=_t(8, 256, 4, dtype=torch.float32)), "v_scale has dtype"),
    (dict(ks=None), "k_scale is required"),
])
def test_decode_rejects_mismatched_tensors(over, msg):
    a = _decode_args(**over)
    with pytest.raises(RuntimeError, match=msg):
        torch.ops.voltattn.decode(a["q"], a["k"], a["v"], a["ks"], a["vs"], "q4+", 32)


def test_decode_f16_and_gqa_checks():
    q = _t(8, 128, dtype=torch.float16)
    kf = _t(8, 100, 128, dtype=torch.float16)
    assert torch.ops.voltattn.decode(q, kf, kf, None, None, "f16+").shape == (8, 128)
    with pytest.raises(RuntimeError, match="k has dtype"):
        torch.ops.voltattn.decode(q, _t(8, 100, 128), _t(8, 100, 128), None, None, "f16+")
    k3 = _t(3, 100, 48)
    s3 = _t(3, 100, 4, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="multiple of K/V heads"):
        torch.ops.voltattn.decode_gqa(q, k3, k3, s3, s3, "q3+")
    with pytest.raises(RuntimeError, match="group must be"):
        torch.ops.voltattn.decode_gqa(q, _t(2, 100, 48), _t(2, 100, 48), s3[:2], s3[:2], "q3+", 48)


def _paged_args(**over):
    a = dict(q=_t(2, 8, 128, dtype=torch.float16), kp=_t(16, 2, 64, 128), vp=_t(16, 2, 64, 128),
             ksp=_t(16, 2, 64, 4, dtype=torch.float16), vsp=_t(16, 2, 64, 4, dtype=torch.float16),
             bt=_t(2, 8, dtype=torch.int32), sl=_t(2, dtype=torch.int32))
    a.update(over)
    return a


@pytest.mark.parametrize("over,msg", [
    (dict(kp=_t(16, 3, 64, 128), vp=_t(16, 3, 64, 128)), "multiple of K/V heads"),
    (dict(vp=_t(16, 2, 64, 64)), "v has shape"),
    (dict(ksp=_t(16, 2, 32, 4, dtype=torch.float16)), "k_scale has shape"),
    (dict(bt=_t(3, 8, dtype=torch.int32)), "block_table must be"),
    (dict(bt=_t(2, 8, dtype=torch.int64)), "block_table has dtype"),
    (dict(sl=_t(3, dtype=torch.int32)), "seq_lens has shape"),
    (dict(q=_t(2, 8, 128, dtype=torch.bfloat16)), "q has dtype"),
])
def test_decode_paged_rejects_mismatched_tensors(over, msg):
    a = _paged_args(**over)
    with pytest.raises(RuntimeError, match=msg):
        torch.ops.voltattn.decode_paged(a["q"], a["kp"], a["vp"], a["ksp"], a["vsp"], a["bt"], a["sl"],
                                        "q8+", 512)


@pytest.mark.parametrize("over,msg", [
    (dict(pages=_t(16, 4, 64, 64)), "pages hold 4 K/V heads"),      # pool Hkv != x's Hkv
    (dict(pages=_t(16, 2, 64, 128)), "pages has shape"),            # q8 rows into a q4 pool
    (dict(scales=_t(16, 2, 64, 2, dtype=torch.float16)), "scale_pages has shape"),
    (dict(x=_t(2, 2, 5, 128, dtype=torch.float32)), "x has dtype"),
    (dict(start=_t(3, dtype=torch.int32)), "start has shape"),
    (dict(bt=_t(2, 8, dtype=torch.int16)), "block_table has dtype"),
])
def test_append_rejects_mismatched_tensors(over, msg):
    a = dict(x=_t(2, 2, 5, 128, dtype=torch.float16), start=_t(2, dtype=torch.int32),
             bt=_t(2, 8, dtype=torch.int32), pages=_t(16, 2, 64, 64),
             scales=_t(16, 2, 64, 4, dtype=torch.float16))
    a.update(over)
    with pytest.raises(RuntimeError, match=msg):
        torch.ops.voltattn.append_kv(a["x"], a["start"], a["bt"], a["pages"], a["scales"], "q4+")


def test_quantize_rejects_bad_arguments():
    with pytest.raises(RuntimeError, match="bits must be"):
        torch.ops.voltattn.quantize(_t(4, 128, dtype=torch.float32), 5, 32)
    with pytest.raises(RuntimeError, match="x must be fp32"):
        torch.ops.voltattn.quantize(_t(4, 128, dtype=torch.float16), 8, 32)
    with pytest.raises(RuntimeError, match="group must be"):
        torch.ops.voltattn.quantize(_t(4, 96, dtype=torch.float32), 8, 64)


def test_dequantize_rejects_bad_arguments():
    sc = _t(4, 4, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="bits must be"):
        torch.ops.voltattn.dequantize(_t(4, 128), sc, 5, 32)
    with pytest.raises(RuntimeError, match="packed must be uint8"):
        torch.ops.voltattn.dequantize(_t(4, 128, dtype=torch.float16), sc, 8, 32)
    with pytest.raises(RuntimeError, match="whole 3-bit codes"):
        torch.ops.voltattn.dequantize(_t(4, 47), sc, 3, 32)
    with pytest.raises(RuntimeError, match="group must be"):
        torch.ops.voltattn.dequantize(_t(4, 48), sc, 4, 64)          # D = 96
    with pytest.raises(RuntimeError, match="scales has shape"):
        torch.ops.voltattn.dequantize(_t(4, 64), _t(4, 2, dtype=torch.float16), 4, 32)
    with pytest.raises(RuntimeError, match="scales has dtype"):
        torch.ops.voltattn.dequantize(_t(4, 64), _t(4, 4, dtype=torch.float32), 4, 32)


def _traced_guards(fn, *args):
    """Guards and symbol values recorded while tracing fn with symbolic shapes."""
    from torch.fx.experimental.proxy_tensor import make_fx
    gm = make_fx(fn, tracing_mode="symbolic")(*args)
    for n in gm.graph.nodes:
        v = n.meta.get("val")
        if hasattr(v, "fake_mode"):
            se = v.fake_mode.shape_env
            return [g.expr for g in se.guards], {k: int(x) for k, x in se.var_to_val.items()}
    raise AssertionError("no fake values traced")


def _free_of(guards, values, sizes):
    """No guard mentions a symbol whose traced value is one of `sizes` (which
    the inputs use only for batch, heads, positions, pages or rows)."""
    syms = {s for s, x in values.items() if x in sizes}
    bad = [g for g in guards if g.free_symbols & syms]
    assert not bad, bad


# Distinct sizes, none equal to D (128), D/G (4) or a row width, so that no
# size shares a symbol with another under duck sizing.
def test_symbolic_shapes_stay_symbolic():
    H, Hkv, L, G = 6, 2, 1000, 32
    q = torch.zeros(H, 128, dtype=torch.float16)
    k = torch.zeros(H, L, 128, dtype=torch.uint8)
    ks = torch.zeros(H, L, 4, dtype=torch.float16)
    g, v = _traced_guards(lambda q, k, v, ks, vs: torch.ops.voltattn.decode(q, k, v, ks, vs, "q8+", G, 0),
                          q, k, k.clone(), ks, ks.clone())
    _free_of(g, v, {H, L})
    k2 = torch.zeros(Hkv, L, 64, dtype=torch.uint8)
    ks2 = torch.zeros(Hkv, L, 4, dtype=torch.float16)
    g, v = _traced_guards(lambda q, k, v, ks, vs: torch.ops.voltattn.decode_gqa(q, k, v, ks, vs, "q4+", G, 0),
                          q, k2, k2.clone(), ks2, ks2.clone())
    _free_of(g, v, {L})                              # H and Hkv: only their divisibility is asserted
    assert not [x for x in g if x.free_symbols and all(str(s) in {str(t) for t, y in v.items() if y == H}
                                                      for s in x.free_symbols)]
    B, P, PR, MP = 3, 10, 256, 5
    qb = torch.zeros(B, H, 128, dtype=torch.float16)
    kp = torch.zeros(P, Hkv, PR, 48, dtype=torch.uint8)
    ksp = torch.zeros(P, Hkv, PR, 4, dtype=torch.float16)
    bt = torch.zeros(B, MP, dtype=torch.int32)
    sl = torch.zeros(B, dtype=torch.int32)
    g, v = _traced_guards(lambda *a: torch.ops.voltattn.decode_paged(*a, "q3+", 1280, G, 0),
                          qb, kp, kp.clone(), ksp, ksp.clone(), bt, sl)
    _free_of(g, v, {B, P, PR, MP})
    x = torch.zeros(B, Hkv, 7, 128, dtype=torch.float16)
    st = torch.zeros(B, dtype=torch.int32)
    kp8 = torch.zeros(P, Hkv, PR, 128, dtype=torch.uint8)
    g, v = _traced_guards(lambda *a: torch.ops.voltattn.append_kv(*a, "q8+", G), x, st, bt, kp8, ksp)
    _free_of(g, v, {B, P, PR, MP, 7})
    g, v = _traced_guards(lambda x: torch.ops.voltattn.quantize(x, 4, G), torch.zeros(5, 9, 128))
    _free_of(g, v, {5, 9})
    g, v = _traced_guards(lambda p, s: torch.ops.voltattn.dequantize(p, s, 3, G),
                          torch.zeros(5, 9, 48, dtype=torch.uint8), torch.zeros(5, 9, 4, dtype=torch.float16))
    _free_of(g, v, {5, 9})
