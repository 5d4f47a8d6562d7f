"""Pins of the CPU oracle's grouped-query and paged forms (oracle/batch.py).

The per-head arithmetic is the reference's reference() (src/voltattn.cu:769-794,
pinned in test_oracle_reference.py); these tests pin what is layered on it:
the query-head -> KV-head mapping (closed forms that a wrong mapping fails, and
an independent float64 brute force) and the page-table addressing (a
hand-laid table and a scatter/gather round trip)."""
import numpy as np
import pytest

import oracle
from oracle import batch


def _f16(x):
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def _brute(kd, vd, q16, Hq, Hkv, L, D):
    """Textbook softmax attention in float64 with query head h on KV head h // (Hq/Hkv)."""
    k = kd.reshape(Hkv, L, D).astype(np.float64)
    v = vd.reshape(Hkv, L, D).astype(np.float64)
    q = q16.view(np.float16).astype(np.float64).reshape(Hq, D)
    out = np.empty((Hq, D))
    g = Hq // Hkv
    for h in range(Hq):
        s = k[h // g] @ q[h] / np.sqrt(D)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ v[h // g]
    return out.ravel()


def test_gqa_equal_heads_is_the_reference():
    rng = np.random.default_rng(1)
    H, L, D = 3, 40, 64
    kd = rng.standard_normal(H * L * D).astype(np.float32)
    vd = rng.standard_normal(H * L * D).astype(np.float32)
    q = _f16(rng.standard_normal(H * D))
    np.testing.assert_array_equal(batch.reference_gqa(kd, vd, q, H, H, L, D),
                                  oracle.reference(kd, vd, q, H, L, D))


def test_gqa_mapping_closed_form():
    # V of KV head j is the constant j+1, so every output of query head h equals
    # (h // (Hq/Hkv)) + 1 whatever K and q are; h % Hkv (a plausible slip) fails.
    Hq, Hkv, L, D = 12, 3, 17, 64
    rng = np.random.default_rng(2)
    kd = rng.standard_normal(Hkv * L * D).astype(np.float32)
    vd = np.repeat(np.arange(1, Hkv + 1, dtype=np.float32), L * D)
    q = _f16(rng.standard_normal(Hq * D))
    out = batch.reference_gqa(kd, vd, q, Hq, Hkv, L, D).reshape(Hq, D)
    want = (np.arange(Hq) // (Hq // Hkv) + 1).astype(np.float32)
    np.testing.assert_allclose(out, np.repeat(want[:, None], D, axis=1), rtol=1e-6)


@pytest.mark.parametrize("Hq,Hkv,L,D", [(8, 2, 33, 64), (14, 2, 5, 128), (6, 6, 1, 64)])
def test_gqa_matches_float64_brute_force(Hq, Hkv, L, D):
    rng = np.random.default_rng(Hq * 100 + L)
    kd = rng.standard_normal(Hkv * L * D).astype(np.float32)
    vd = rng.standard_normal(Hkv * L * D).astype(np.float32)
    q = _f16(rng.standard_normal(Hq * D))
    got = batch.reference_gqa(kd, vd, q, Hq, Hkv, L, D)
    np.testing.assert_allclose(got, _brute(kd, vd, q, Hq, Hkv, L, D), rtol=1e-6, atol=1e-7)


def test_paged_addressing_hand_laid():
    # 2 KV heads, page_rows 4, one row = 1 value equal to its (head, position) id
    Hkv, P, L = 2, 4, 10
    rows = np.array([[[100 * h + j] for j in range(L)] for h in range(Hkv)], np.int32)
    table = np.array([5, 0, 3])              # positions 0-3 -> page 5, 4-7 -> 0, 8-9 -> 3
    pool = np.full((6, Hkv, P, 1), -1, np.int32)
    batch.scatter_rows(pool, rows, table, P)
    assert pool[5, 1, 2, 0] == 102           # head 1, position 2
    assert pool[0, 0, 3, 0] == 7             # head 0, position 7
    assert pool[3, 1, 1, 0] == 109           # head 1, position 9
    assert pool[3, 0, 2, 0] == -1            # past L: untouched
    assert np.all(pool[[1, 2, 4]] == -1)     # pages outside the table: untouched
    np.testing.assert_array_equal(batch.gather_rows(pool, table, L, P), rows)


def test_paged_round_trip_random():
    rng = np.random.default_rng(7)
    Hkv, P, W = 3, 8, 5
    for L in (1, 7, 8, 9, 64, 77):
        npg = -(-L // P)
        table = rng.permutation(npg + 4)[:npg]
        pool = rng.integers(0, 255, (npg + 4, Hkv, P, W), dtype=np.uint8)
        rows = rng.integers(0, 255, (Hkv, L, W), dtype=np.uint8)
        batch.scatter_rows(pool, rows, table, P)
        np.testing.assert_array_equal(batch.gather_rows(pool, table, L, P), rows)


def _draw(Hkv, L, D, seed, positive=False):
    rng = np.random.default_rng(seed)
    kd = rng.standard_normal((Hkv, L, D)).astype(np.float32)
    vd = rng.standard_normal((Hkv, L, D)).astype(np.float32)
    if positive:
        vd = np.abs(vd) + np.arange(Hkv, dtype=np.float32)[:, None, None]   # heads differ by offset
    return kd, vd


@pytest.mark.parametrize("Hq,Hkv,L,D", [(4, 2, 37, 64), (6, 3, 300, 128), (2, 2, 5, 128)])
def test_magnitude_is_the_reference_for_nonnegative_v(Hq, Hkv, L, D):
    # sum_j p_j |v_jd| = sum_j p_j v_jd when V >= 0: the same weights and head mapping as reference()
    kd, vd = _draw(Hkv, L, D, 0xA11 + L, positive=True)
    q = _f16(np.random.default_rng(L).standard_normal((Hq, D)))
    mag = batch.magnitude_gqa(kd, vd, q, Hq, Hkv, L, D)
    ref = batch.reference_gqa(kd, vd, q, Hq, Hkv, L, D).astype(np.float64)
    np.testing.assert_allclose(mag, ref, rtol=2e-6)


def test_magnitude_bounds_the_reference_and_closed_forms():
    Hq, Hkv, L, D = 6, 2, 200, 64
    kd, vd = _draw(Hkv, L, D, 0xA12)
    q = _f16(np.random.default_rng(7).standard_normal((Hq, D)))
    mag = batch.magnitude_gqa(kd, vd, q, Hq, Hkv, L, D)
    ref = batch.reference_gqa(kd, vd, q, Hq, Hkv, L, D).astype(np.float64)
    assert np.all(mag >= np.abs(ref) - 1e-6 * mag)
    assert np.mean(mag > 2 * np.abs(ref)) > 0.2            # signed V cancels: the bound is not |ref|
    # one position: the weight is 1, so the magnitude is |v_0| exactly
    mag1 = batch.magnitude_gqa(kd[:, :1], vd[:, :1], q, Hq, Hkv, 1, D).reshape(Hq, D)
    np.testing.assert_array_equal(mag1, np.abs(np.repeat(vd[:, 0], Hq // Hkv, axis=0)).astype(np.float64))


def test_cancelling_case_has_no_headroom_under_the_plain_bound():
    """The fixed grouped case of tests/test_gpu_fuzz.py::test_cancelling_grouped_case
    (q4+, Hq 7 over Hkv 1, L 16): an ideal fp32 kernel (exact dot products,
    fp32 scores in log2 units, fp32 exp2, sequential fp32 sums, fp16 output)
    already lands within 5% of the plain fp16 rounding bound, because outputs
    cancel >1000x below sum_j p_j |v_jd|; cond_bound's widening (8 fp32 ulps of
    that magnitude) is what any fp32 summation order needs there."""
    import voltattn_amd as va
    from tests import batch_util
    from tests.numerics import cond_bound, tight_bound
    case, fmt, Hkv, Hq, L, D, G = 503, va.Fmt.Q4M, 1, 7, 16, 128, 32
    c = batch_util.kv_case(fmt, Hkv, L, D, G, 0xB000 + case)
    q = batch_util.queries(Hq, D, 0xB100 + case)
    ref = batch.reference_gqa(c["kd"], c["vd"], q, Hq, Hkv, L, D).astype(np.float64).reshape(Hq, D)
    mag = np.asarray(batch.magnitude_gqa(c["kd"], c["vd"], q, Hq, Hkv, L, D), np.float64).reshape(Hq, D)
    kd = c["kd"].reshape(L, D).astype(np.float64)
    vd = c["vd"].reshape(L, D).astype(np.float32)
    qq = q.view(np.float16).reshape(Hq, D).astype(np.float64)
    out = np.zeros((Hq, D))
    for h in range(Hq):
        s2 = (kd @ qq[h] * (np.log2(np.e) / np.sqrt(D))).astype(np.float32)
        p = np.exp2(s2 - s2.max()).astype(np.float32)
        l, o = np.float32(0), np.zeros(D, np.float32)
        for j in range(L):
            l = np.float32(l + p[j])
            o = (o + p[j] * vd[j]).astype(np.float32)
        out[h] = (o / l).astype(np.float16)
    ratio = np.max(np.abs(out - ref) / tight_bound(ref))
    assert 0.95 < ratio <= 1.0
    assert np.max(mag / np.maximum(np.abs(ref), 1e-30)) > 1000
    assert np.all(np.abs(out - ref) <= cond_bound(ref, mag))
