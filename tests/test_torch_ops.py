"""The torch.library binding without a GPU: the ops are registered under
torch.ops.voltattn, their fake (meta) implementations give the documented
output shapes, and CPU tensors are refused loudly (no CPU fallback)."""
import pytest
import torch

import voltattn_amd.torch_ops  # noqa: F401  (registers torch.ops.voltattn.*)


def test_ops_registered():
    for name in ("decode", "decode_gqa", "decode_paged", "append_kv", "quantize"):
        assert hasattr(torch.ops.voltattn, name), name


def test_fake_shapes_on_meta():
    m = dict(device="meta")
    q = torch.empty(32, 128, dtype=torch.float16, **m)
    k = torch.empty(8, 4096, 128, dtype=torch.uint8, **m)
    s = torch.empty(8, 4096, 4, dtype=torch.float16, **m)
    assert torch.ops.voltattn.decode_gqa(q, k, k, s, s, "q8+").shape == (32, 128)
    assert torch.ops.voltattn.decode(q, torch.empty(32, 4096, 128, dtype=torch.uint8, **m), k, s, s,
                                     "q8+").shape == (32, 128)
    qb = torch.empty(4, 32, 128, dtype=torch.float16, **m)
    pages = torch.empty(64, 8, 256, 64, dtype=torch.uint8, **m)
    sp = torch.empty(64, 8, 256, 4, dtype=torch.float16, **m)
    bt = torch.empty(4, 16, dtype=torch.int32, **m)
    sl = torch.empty(4, dtype=torch.int32, **m)
    out = torch.ops.voltattn.decode_paged(qb, pages, pages, sp, sp, bt, sl, "q4+", 4096)
    assert out.shape == (4, 32, 128) and out.dtype == torch.float16
    packed, scales = torch.ops.voltattn.quantize(torch.empty(10, 128, **m), 3, 32)
    assert packed.shape == (10, 48) and scales.shape == (10, 4)


def test_cpu_tensors_refused():
    q = torch.zeros(4, 128, dtype=torch.float16)
    k = torch.zeros(4, 64, 128, dtype=torch.uint8)
    s = torch.zeros(4, 64, 4, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="gfx950"):
        torch.ops.voltattn.decode(q, k, k, s, s, "q8+")
    with pytest.raises(RuntimeError, match="gfx950"):
        torch.ops.voltattn.quantize(torch.zeros(2, 128), 8, 32)
