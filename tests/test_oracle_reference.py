"""Pins of the oracle's double-precision attention (reference(),
src/voltattn.cu:769-794) and of the split-L log-sum-exp algebra
(src/voltattn.cu:80-120, 651-672):

* equality with scipy's softmax followed by a float64 matrix-vector product;
* closed forms: identical K rows give the mean of the V rows; one dominant
  score selects its V row; L = 1 returns the single V row;
* the split-L merge equals the unsplit reference for every split count,
  including splits that are empty (S > L, ceil(L/S) * (S-1) >= L).
"""
import numpy as np
import pytest
from scipy.special import softmax

import oracle


def _rand(H, L, D, seed):
    rng = np.random.default_rng(seed)
    kd = rng.standard_normal(H * L * D).astype(np.float32)
    vd = rng.standard_normal(H * L * D).astype(np.float32)
    q = rng.standard_normal(H * D).astype(np.float16).view(np.uint16)
    return kd, vd, q


@pytest.mark.parametrize("H,L,D", [(2, 37, 64), (3, 129, 128), (1, 1000, 128)])
def test_reference_matches_scipy_softmax(H, L, D):
    kd, vd, q = _rand(H, L, D, H * L)
    out = oracle.reference(kd, vd, q, H, L, D)
    K = kd.reshape(H, L, D).astype(np.float64)
    V = vd.reshape(H, L, D).astype(np.float64)
    Q = q.view(np.float16).astype(np.float64).reshape(H, D)
    for h in range(H):
        p = softmax(K[h] @ Q[h] / np.sqrt(D))
        np.testing.assert_allclose(out[h * D:(h + 1) * D], (p @ V[h]).astype(np.float32),
                                   rtol=1e-6, atol=1e-7)


def test_identical_keys_give_mean_of_values():
    H, L, D = 2, 50, 64
    kd, vd, q = _rand(H, L, D, 3)
    kd = np.tile(kd.reshape(H, L, D)[:, :1, :], (1, L, 1)).ravel()
    out = oracle.reference(kd, vd, q, H, L, D)
    np.testing.assert_allclose(out, vd.reshape(H, L, D).astype(np.float64).mean(axis=1).ravel(),
                               rtol=1e-6, atol=1e-7)


def test_dominant_score_selects_its_row():
    H, L, D = 1, 40, 64
    kd, vd, q = _rand(H, L, D, 4)
    qf = q.view(np.float16).astype(np.float32)
    K = kd.reshape(L, D)
    K[17] = 1000.0 * np.sign(qf)            # score of row 17 exceeds the others by >> 40
    out = oracle.reference(K.ravel(), vd, q, H, L, D)
    np.testing.assert_allclose(out, vd.reshape(L, D)[17], rtol=1e-6, atol=1e-7)


def test_single_position_returns_its_value_row():
    H, L, D = 3, 1, 128
    kd, vd, q = _rand(H, L, D, 5)
    np.testing.assert_array_equal(oracle.reference(kd, vd, q, H, L, D), vd)


@pytest.mark.parametrize("S", [1, 2, 3, 5, 9, 13, 40])
def test_split_merge_equals_unsplit(S):
    H, L, D = 2, 13, 64
    kd, vd, q = _rand(H, L, D, 6)
    ref = oracle.reference(kd, vd, q, H, L, D)
    out, lse, avg = oracle.split_attention(kd, vd, q, H, L, D, S)
    np.testing.assert_allclose(out, ref, rtol=1e-6, atol=1e-7)
    chunk = -(-L // S)
    for s in range(S):
        empty = min(L, s * chunk) >= min(L, s * chunk + chunk)
        assert np.isneginf(lse[:, s]).all() == empty


def test_split_partials_are_split_softmax():
    H, L, D, S = 1, 20, 64, 3
    kd, vd, q = _rand(H, L, D, 8)
    _, lse, avg = oracle.split_attention(kd, vd, q, H, L, D, S)
    K = kd.reshape(L, D).astype(np.float64)
    V = vd.reshape(L, D).astype(np.float64)
    sc = K @ q.view(np.float16).astype(np.float64) / np.sqrt(D)
    chunk = -(-L // S)
    for s in range(S):
        sl = slice(s * chunk, min(L, (s + 1) * chunk))
        np.testing.assert_allclose(lse[0, s], np.log(np.exp(sc[sl]).sum()), rtol=1e-12)
        np.testing.assert_allclose(avg[0, s], softmax(sc[sl]) @ V[sl], rtol=1e-9, atol=1e-12)
