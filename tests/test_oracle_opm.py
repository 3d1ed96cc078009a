"""Pins the float64 outer-product-mean oracle (oracle/opm.py) against per-element brute-force
sums, closed-form special cases, the reference test's einsum statement of opm_outer's rounding
(tests/test_opm.py:82-86 of the reference), a hand-fixed rounding case, and the identity that
links the two kernels. CPU only.
"""
import numpy as np

from oracle import opm


def rand16(rng, *shape, s=1.0):
    return (rng.standard_normal(shape) * s).astype(np.float16).astype(np.float64)


def test_opm_update_brute_force():
    rng = np.random.default_rng(0)
    B, K, D, F = 3, 32, 2, 16
    lhs, t = rand16(rng, B, K), rand16(rng, K, D, F)
    bias = rng.standard_normal(F).astype(np.float32)
    norm = rng.integers(1, 4, size=(B, D)).astype(np.float32)
    res = rand16(rng, B, D, F)
    got = opm.opm_update(lhs, t, bias, norm, 1e-3, res)
    for b in range(B):
        for d in range(D):
            for f in range(F):
                s = sum(lhs[b, k] * t[k, d, f] for k in range(K))
                want = (s + float(bias[f])) / (1e-3 + float(norm[b, d])) + res[b, d, f]
                assert abs(got[b, d, f] - want) < 1e-12
    # without a residual nothing is added
    np.testing.assert_allclose(opm.opm_update(lhs, t, bias, norm, 1e-3) + res, got, rtol=0, atol=1e-12)


def test_opm_update_special_cases():
    rng = np.random.default_rng(1)
    B, K, D, F = 5, 64, 3, 32
    lhs, t = rand16(rng, B, K), rand16(rng, K, D, F)
    # zero bias, unit norm, zero eps: the plain GEMM over the flattened [K, D F] operand
    got = opm.opm_update(lhs, t, np.zeros(F), np.ones((B, D)), 0.0)
    np.testing.assert_allclose(got.reshape(B, D * F), np.matmul(lhs, t.reshape(K, D * F)), rtol=1e-12)
    # zero lhs: bias / (eps + norm), the norm indexed by (b, d) and the bias by f
    bias = rng.standard_normal(F)
    norm = rng.integers(1, 9, size=(B, D)).astype(np.float64)
    got = opm.opm_update(np.zeros((B, K)), t, bias, norm, 0.5)
    for b in range(B):
        for d in range(D):
            np.testing.assert_allclose(got[b, d], bias / (0.5 + norm[b, d]), rtol=1e-14)


def test_opm_outer_brute_force():
    rng = np.random.default_rng(2)
    B, C, D, F = 2, 3, 2, 16
    left, right = rand16(rng, 16, B, C), rand16(rng, 16, D, 32)
    wT = rand16(rng, F, C * 32, s=0.1)
    got = opm.opm_outer(left, right, wT)
    for b in range(B):
        for d in range(D):
            for f in range(F):
                s = 0.0
                for c in range(C):
                    for e in range(32):
                        g = sum(left[a, b, c] * right[a, d, e] for a in range(16))
                        s += float(np.float16(g)) * wT[f, c * 32 + e]
                assert abs(got[b, d, f] - s) < 1e-9


def test_opm_outer_matches_reference_test_statement():
    """The reference test's float32 restatement: einsum('abc,ade->bced') rounded to f16, reshaped
    to [B, C E, D], then einsum('bkd,kf->bdf') with w = wT^T."""
    rng = np.random.default_rng(3)
    B, C, D, F = 7, 32, 8, 64
    left, right = rand16(rng, 16, B, C), rand16(rng, 16, D, 32)
    wT = rand16(rng, F, C * 32, s=1 / 32)
    act = np.einsum("abc,ade->bced", left, right).astype(np.float16).astype(np.float64)
    act = act.reshape(B, C * 32, D)
    want = np.einsum("bkd,kf->bdf", act, wT.T)
    np.testing.assert_allclose(opm.opm_outer(left, right, wT), want, rtol=1e-12, atol=1e-12)


def test_opm_outer_rounds_the_outer_product():
    """g = 1 + 2^-12 on even e and 1 on odd e, weights +1 / -1: rounding g to fp16 (1 + 2^-12
    rounds to 1) cancels every pair and gives 0; keeping it gives 16 C 2^-12."""
    B, C, D, F = 1, 16, 1, 16
    left = np.zeros((16, B, C))
    left[0] = 1.0
    left[1] = 2.0 ** -12
    right = np.zeros((16, D, 32))
    right[0] = 1.0
    right[1, :, 0::2] = 1.0  # the second row adds 2^-12 on even e only
    wT = np.tile(np.where(np.arange(32) % 2 == 0, 1.0, -1.0), C)[None, :].repeat(F, 0)
    assert np.all(opm.opm_outer(left, right, wT, round_mid=True) == 0.0)
    np.testing.assert_allclose(opm.opm_outer(left, right, wT, round_mid=False), 16 * C * 2.0 ** -12)


def test_update_and_outer_agree():
    """opm_update on lhs[b, (a, c)] = left[a, b, c] and t[(a, c), d, f] = sum_e right[a, d, e]
    wT[f, c E + e] is the same contraction as opm_outer, without the rounding of g."""
    rng = np.random.default_rng(4)
    B, C, D, F = 6, 16, 4, 32
    left, right = rand16(rng, 16, B, C), rand16(rng, 16, D, 32)
    wT = rand16(rng, F, C * 32, s=0.1)
    lhs = left.transpose(1, 0, 2).reshape(B, 16 * C)
    w = wT.T.reshape(C, 32, F)
    t = np.einsum("ade,cef->acdf", right, w).reshape(16 * C, D, F)
    got = opm.opm_update(lhs, t, np.zeros(F), np.ones((B, D)), 0.0)
    np.testing.assert_allclose(got, opm.opm_outer(left, right, wT, round_mid=False), rtol=1e-10, atol=1e-12)
