"""VoltaLayerNorm and VoltaGdp on gfx950 against the float64 oracle, through the C ABI.

The reference checks them against jnp LayerNorm and the gated dual projection
(tests/test_fused.py:151-178). Tolerance (fp16 outputs): the absolute error beyond each output's
fp16 half-ulp rounding is at most 2e-3 at unit-scale inputs.
"""
import numpy as np
import pytest
import torch

from conftest import abs_excess
from oracle import fused as orf

pytestmark = pytest.mark.gpu
ATOL = 2e-3


def f16(a):
    return np.asarray(a, np.float16)


def dev(*xs):
    return [torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in xs]


@pytest.mark.parametrize("m,c", [(1000, 64), (37, 128), (300, 256), (5, 8), (64, 24), (33, 100), (7, 1),
                                 (2, 512)])
def test_layer_norm(hip, m, c):
    rng = np.random.default_rng(m * 1000 + c)
    x = f16(rng.standard_normal((m, c)) * 2 + 0.3)
    sc = (1 + 0.1 * rng.standard_normal(c)).astype(np.float32)
    of = (0.1 * rng.standard_normal(c)).astype(np.float32)
    tx, tsc, tof = dev(x, sc, of)
    out = hip.layer_norm(tx, tsc, tof, 1e-5).float().cpu().numpy()
    ref = orf.layer_norm_onepass(x, sc, of, 1e-5)
    assert abs_excess(out, ref, fp16_out=True) <= ATOL


def test_layer_norm_constant_rows(hip):
    """var = max(E[x^2] - mean^2, 0): a constant row gives exactly the offset."""
    x = np.full((4, 128), 2.5, np.float16)
    sc = np.ones(128, np.float32)
    of = np.linspace(-1, 1, 128).astype(np.float32)
    out = hip.layer_norm(*dev(x, sc, of)).float().cpu().numpy()
    assert abs_excess(out, np.broadcast_to(of, (4, 128)), fp16_out=True) <= 1e-3


# K in {64, 128} with N in {64, 128, 256} take the persistent kernel; 20000 rows give each of its
# workgroups several tiles and end in a 32-row tile
@pytest.mark.parametrize("m,k,n", [(100, 64, 128), (300, 128, 64), (1, 64, 8), (130, 37, 72), (64, 256, 256),
                                   (20000, 128, 256), (4100, 64, 64), (70, 128, 128), (129, 64, 256)])
@pytest.mark.parametrize("act", [0, 1])
def test_gated_dual_proj(hip, m, k, n, act):
    rng = np.random.default_rng(m + k + n + act)
    x = f16(rng.standard_normal((m, k)))
    wp = f16(rng.standard_normal((k, n)) * k ** -0.5)
    wg = f16(rng.standard_normal((k, n)) * k ** -0.5)
    bp, bg = f16(rng.standard_normal(n) * 0.1), f16(rng.standard_normal(n) * 0.1)
    mask = f16(rng.choice([1.0, 0.0, 0.5, -1.0], size=m))
    out = hip.gated_dual_proj(*dev(x, wp, bp, wg, bg, mask), activation=act).float().cpu().numpy()
    ref = orf.gated_dual_proj(x, wp, bp, wg, bg, mask, act)
    assert abs_excess(out, ref, fp16_out=True) <= ATOL


def test_gated_dual_proj_rejections(hip):
    x, w, b, mask = (torch.zeros(s, dtype=torch.float16, device="cuda") for s in ((4, 16), (16, 12), (12,), (4,)))
    with pytest.raises(hip.InvalidArgument, match="N must be a multiple of 8"):
        hip.gated_dual_proj(x, w, b, w, b, mask)
    w, b = torch.zeros((16, 16), dtype=torch.float16, device="cuda"), torch.zeros(16, dtype=torch.float16, device="cuda")
    with pytest.raises(hip.InvalidArgument, match=r"activation is 0 \(sigmoid\) or 1 \(swish\), got 3"):
        hip.gated_dual_proj(x, w, b, w, b, mask, activation=3)
