"""VoltaOpmUpdate and VoltaOpmOuter on gfx950 against the float64 oracle, through the C ABI.

The reference's own cases (tests/test_opm.py:92-140): opm_update at B 1, 37 and 260, D 4, 64 and
260, K 32, 64 and 512, F 128 and 64, with and without the residual, t scaled by K^-1/2, the norm
an integer count in [1, K/32]; opm_outer at the same B and D on 16 rows with 32 channels and
w scaled by 1/32. Tolerance (fp16 outputs): the absolute error beyond each output's fp16 half-ulp
rounding is at most 2e-3 (the reference's 2e-3 relative bound at these unit-scale outputs).
"""
import numpy as np
import pytest
import torch

from conftest import abs_excess
from oracle import opm as oro

pytestmark = pytest.mark.gpu
ATOL = 2e-3


def dev(*xs):
    return [torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in xs]


def update_inputs(seed, b, k, d, f):
    rng = np.random.default_rng(seed)
    lhs = rng.standard_normal((b, k)).astype(np.float16)
    t = (rng.standard_normal((k, d, f)) * k ** -0.5).astype(np.float16)
    bias = (rng.standard_normal(f) * 0.1).astype(np.float32)
    norm = rng.integers(1, k // 32 + 1, size=(b, d)).astype(np.float32)
    res = (rng.standard_normal((b, d, f)) * 2).astype(np.float16)
    return lhs, t, bias, norm, res


UPDATE_CASES = ([(b, 64, d, 128) for b in (1, 37, 260) for d in (4, 64, 260)] +
                [(37, k, 64, f) for k in (32, 512) for f in (128, 64)] +
                [(260, 512, 260, 64), (37, 64, 64, 64), (5, 96, 9, 16), (70, 32, 3, 32)])


@pytest.mark.parametrize("b,k,d,f", UPDATE_CASES)
@pytest.mark.parametrize("residual", [False, True])
def test_opm_update(hip, b, k, d, f, residual):
    lhs, t, bias, norm, res = update_inputs(b * 7 + k * 3 + d + f, b, k, d, f)
    tl, tt, tb, tn, tr = dev(lhs, t, bias, norm, res)
    out = hip.opm_update(tl, tt, tb, tn, tr if residual else None, eps=1e-3)
    ref = oro.opm_update(lhs, t, bias, norm, 1e-3, res if residual else None)
    assert abs_excess(out.float().cpu().numpy(), ref) <= ATOL


def test_opm_update_in_place_residual(hip):
    """The residual may be the output buffer itself; a separate residual is left as it was."""
    lhs, t, bias, norm, res = update_inputs(11, 37, 64, 64, 128)
    tl, tt, tb, tn, tr = dev(lhs, t, bias, norm, res)
    ref = oro.opm_update(lhs, t, bias, norm, 1e-3, res)
    before = tr.clone()
    separate = hip.opm_update(tl, tt, tb, tn, tr, eps=1e-3)
    assert torch.equal(tr, before)
    inplace = hip.opm_update(tl, tt, tb, tn, tr, eps=1e-3, out=tr)
    assert inplace.data_ptr() == tr.data_ptr()
    assert torch.equal(inplace, separate)
    assert abs_excess(inplace.float().cpu().numpy(), ref) <= ATOL


def outer_inputs(seed, b, c, d, f):
    rng = np.random.default_rng(seed)
    left = rng.standard_normal((16, b, c)).astype(np.float16)
    right = rng.standard_normal((16, d, 32)).astype(np.float16)
    wT = (rng.standard_normal((f, 32 * c)) / 32).astype(np.float16)
    return left, right, wT


OUTER_CASES = ([(b, 32, d, f) for b in (1, 37, 260) for d in (4, 64, 260) for f in (128, 64)] +
               [(37, 16, 8, 16), (20, 48, 12, 32), (300, 64, 16, 128)])


@pytest.mark.parametrize("b,c,d,f", OUTER_CASES)
def test_opm_outer(hip, b, c, d, f):
    left, right, wT = outer_inputs(b * 5 + c + d * 3 + f, b, c, d, f)
    out = hip.opm_outer(*dev(left, right, wT))
    ref = oro.opm_outer(left, right, wT)
    assert abs_excess(out.float().cpu().numpy(), ref) <= ATOL


def test_opm_outer_rounds_the_outer_product(hip):
    """g = 1 + 2^-12 on even e and 1 on odd e against weights +1 / -1: the kernel rounds g to
    fp16 (to 1) before the second contraction, so every pair cancels and the output is 0
    exactly; without that rounding it would be 16 C 2^-12 = 1/16."""
    b, c, d, f = 16, 16, 4, 16
    left = np.zeros((16, b, c), np.float16)
    left[0] = 1.0
    left[1] = 2.0 ** -12
    right = np.zeros((16, d, 32), np.float16)
    right[0] = 1.0
    right[1, :, 0::2] = 1.0
    wT = np.tile(np.where(np.arange(32) % 2 == 0, 1.0, -1.0), c)[None, :].repeat(f, 0).astype(np.float16)
    out = hip.opm_outer(*dev(left, right, wT)).float().cpu().numpy()
    assert np.all(out == 0.0)
    assert np.all(oro.opm_outer(left, right, wT, round_mid=False) == 1 / 16)


def test_update_and_outer_agree(hip):
    """opm_update on the row-major regrouping of opm_outer's operands computes the same
    contraction; the two kernels then differ only by opm_outer's fp16 rounding of g."""
    b, c, d, f = 37, 32, 64, 128
    left, right, wT = outer_inputs(5, b, c, d, f)
    lhs = left.transpose(1, 0, 2).reshape(b, 16 * c)
    t = np.einsum("ade,cef->acdf", right.astype(np.float64),
                  wT.astype(np.float64).T.reshape(c, 32, f)).reshape(16 * c, d, f).astype(np.float16)
    out_u = hip.opm_update(*dev(lhs, t, np.zeros(f, np.float32), np.ones((b, d), np.float32)), eps=0.0)
    out_o = hip.opm_outer(*dev(left, right, wT))
    ref = oro.opm_outer(left, right, wT, round_mid=False)
    scale = np.abs(ref).max()
    assert np.abs(out_u.float().cpu().numpy() - out_o.float().cpu().numpy()).max() <= 4e-3 * scale


def test_empty_problems(hip):
    z = hip.opm_update(*dev(np.zeros((0, 64), np.float16), np.zeros((64, 8, 128), np.float16),
                            np.zeros(128, np.float32), np.zeros((0, 8), np.float32)))
    assert z.shape == (0, 8, 128)
    z = hip.opm_outer(*dev(np.zeros((16, 5, 32), np.float16), np.zeros((16, 0, 32), np.float16),
                           np.zeros((64, 1024), np.float16)))
    assert z.shape == (5, 0, 64)


def test_rejections(hip):
    lhs, t, bias, norm, _ = dev(*update_inputs(1, 4, 64, 8, 128))
    with pytest.raises(hip.InvalidArgument, match="K must be a multiple of 32"):
        hip.opm_update(lhs[:, :48].contiguous(), t[:48].contiguous(), bias, norm)
    left, right, wT = dev(*outer_inputs(1, 8, 32, 6, 64))
    with pytest.raises(hip.InvalidArgument, match="D a multiple of 4"):
        hip.opm_outer(left, right, wT)
