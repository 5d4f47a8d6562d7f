"""The correctness gates are not vacuous: mistakes planted in the oracle's own
data on the CPU, of the kind a kernel bug produces, fail them. Gross mistakes
(scrambled codes, a corrupted scale) fail the reference's own rule
|got - ref| <= 3e-3 + 2e-2|ref| (src/voltattn.cu:903); subtle ones (a scale
read from the neighbouring group, a wrong group size, a dropped position) fail
the tight per-element rule the GPU tests also apply (tests/numerics.py)."""
import numpy as np

import oracle
from tests.numerics import tight_bound

H, L, D, S = 8, 257, 128, 3


def _case(bits=8, G=64):
    return oracle.make_case(bits, H, L, D, G, oracle.selftest_seed(H, L, D, S))


def _out_with_v(c, vd):
    return oracle.reference(c["kd"], vd, c["q"], H, L, D).astype(np.float16).astype(np.float64)


def _tight_fails(got, ref):
    return bool(np.any(np.abs(got - ref) > tight_bound(ref)))


def test_neighbouring_group_scale_fails_tight_gate():
    c = _case()
    vd_bad = oracle.dequant(c["vpay"], np.roll(c["vsc"], 1), H * L, D, 64, 8)
    assert _tight_fails(_out_with_v(c, vd_bad), c["ref"].astype(np.float64))


def test_wrong_group_size_fails_tight_gate():
    c = _case(G=32)
    # G=32 payload read with one scale per 64 elements (every other scale)
    vd_bad = oracle.dequant(c["vpay"], c["vsc"][::2].copy(), H * L, D, 64, 8)
    assert _tight_fails(_out_with_v(c, vd_bad), c["ref"].astype(np.float64))


def test_dropped_tail_position_fails_tight_gate():
    c = _case()
    kd = c["kd"].reshape(H, L, D)[:, : L - 1].ravel()
    vd = c["vd"].reshape(H, L, D)[:, : L - 1].ravel()
    got = oracle.reference(kd, vd, c["q"], H, L - 1, D).astype(np.float16).astype(np.float64)
    assert _tight_fails(got, c["ref"].astype(np.float64))


def test_swapped_nibbles_fail_reference_gate():
    c = _case(bits=4)
    vpay = ((c["vpay"] & 0x0F) << 4) | (c["vpay"] >> 4)      # high/low nibble order reversed
    vd_bad = oracle.dequant(vpay, c["vsc"], H * L, D, 64, 4)
    ok, _ = oracle.gate(_out_with_v(c, vd_bad), c["ref"])
    assert not ok


def test_corrupted_scale_fails_reference_gate():
    c = _case()
    vsc = c["vsc"].copy()
    vsc[::2] = np.float16(8.0).view(np.uint16)
    vd_bad = oracle.dequant(c["vpay"], vsc, H * L, D, 64, 8)
    ok, _ = oracle.gate(_out_with_v(c, vd_bad), c["ref"])
    assert not ok


def test_correct_inputs_pass_both_gates():
    c = _case()
    got = c["ref"].astype(np.float16).astype(np.float64)
    ref = c["ref"].astype(np.float64)
    assert oracle.gate(got, ref)[0]
    assert not _tight_fails(got, ref)
