"""BASELINE config C4 at its own size: the five fused pair-stack ops over M = 262144 rows (N_res =
512) at widths c = 64 and 128, with the shapes bench.py times, against the float64 oracle, in
fp16 and in bf16 activations.

  ln_gdp            two c -> c gated projections (P = 2c), channel-major results, mask of ones
  trimul_epilogue   x_cm [c, M] fp32, c -> c gated output projection
  ln_projection     n = 512 columns (4 slots x 4 heads x 32) and 4 head-bias rows
  output_projection K = 128 -> c with a residual
  transition        hidden width 4c (and 2c at c = 64), with and without add_input

At M = 262144 every persistent workgroup of these kernels walks several row tiles, so the
steady state of each tile loop (the prefetched next tile, the stores of the previous one) runs
here at the exact size the bench measures; the smaller parity tests reach it only in part.
Tolerances are those of tests/test_fused_gpu.py (fp16) and tests/test_fused_bf16_gpu.py (bf16).
"""
import zlib

import numpy as np
import pytest
import torch

from conftest import abs_excess, rel
from oracle import fused as orf

pytestmark = pytest.mark.gpu

M = 262144
EPS = 1e-5
ATOL = 2e-3
REL = 0.02


def rng_for(*key):
    return np.random.default_rng(zlib.crc32(repr(key).encode()))


def acts(rng, bf16, *shape, s=1.0):
    """Activation values (float64, exactly representable in the activation type) and the
    tensor on the GPU."""
    a = rng.standard_normal(shape) * s
    t = torch.from_numpy(a).to(torch.bfloat16 if bf16 else torch.float16)
    return t.double().numpy(), t.cuda()


def f16(rng, *shape, s=1.0):
    return (rng.standard_normal(shape) * s).astype(np.float16)


def f32(rng, *shape, s=1.0, mean=0.0):
    return (rng.standard_normal(shape) * s + mean).astype(np.float32)


def cu(*xs):
    return [torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in xs]


def check(got_t, want, label, bf16):
    torch.cuda.synchronize()
    got = got_t.double().cpu().numpy()
    if bf16:
        tol = ATOL + 2.0 ** -22 * float(np.nanmax(np.abs(want), initial=0.0))
        e = abs_excess(got, want, bf16_out=True)
    else:
        tol = ATOL
        e = abs_excess(got, want)
    r = rel(got, want)
    print("%s: abs excess %.2e rel %.2e" % (label, e, r), flush=True)
    assert e <= tol and r < REL, "%s: abs excess %.2e (tol %.1e), rel %.2e" % (label, e, tol, r)


WIDTHS = (64, 128)
TYPES = ("f16", "bf16")


@pytest.mark.parametrize("dt", TYPES)
@pytest.mark.parametrize("c", WIDTHS)
def test_c4_ln_projection(hip, c, dt):
    rng = rng_for("c4 proj", c, dt)
    x, tx = acts(rng, dt == "bf16", M, c)
    sc, of = f32(rng, c, s=.1, mean=1.), f32(rng, c, s=.1)
    wT, wbT = f16(rng, 512, c, s=c ** -.5), f16(rng, 4, c, s=c ** -.5)
    p, b = hip.ln_projection(tx, *cu(sc, of, wT, wbT), eps=EPS)
    wp, wb = orf.ln_projection(x, sc, of, wT, wbT, None, EPS)
    check(p, wp, "C4 ln_projection c=%d %s p" % (c, dt), dt == "bf16")
    check(b, wb, "C4 ln_projection c=%d %s bias" % (c, dt), dt == "bf16")


@pytest.mark.parametrize("dt", TYPES)
@pytest.mark.parametrize("c", WIDTHS)
def test_c4_output_projection(hip, c, dt):
    rng = rng_for("c4 out", c, dt)
    o, to = acts(rng, dt == "bf16", M, 128)
    r, tr = acts(rng, dt == "bf16", M, c)
    wT, b = f16(rng, c, 128, s=128 ** -.5), f16(rng, c, s=.1)
    out = hip.output_projection(to, *cu(wT, b), residual=tr)
    check(out, orf.output_projection(o, wT, b, r, None), "C4 output_projection c=%d %s" % (c, dt),
          dt == "bf16")


@pytest.mark.parametrize("dt", TYPES)
@pytest.mark.parametrize("c", WIDTHS)
def test_c4_ln_gdp(hip, c, dt):
    rng = rng_for("c4 gdp", c, dt)
    x, tx = acts(rng, dt == "bf16", M, c)
    sc, of = f32(rng, c, s=.1, mean=1.), f32(rng, c, s=.1)
    wpT, wgT = f16(rng, 2 * c, c, s=c ** -.5), f16(rng, 2 * c, c, s=c ** -.5)
    bp, bg = f16(rng, 2 * c, s=.1), f16(rng, 2 * c, s=.1)
    mask = np.ones(M, np.float16)
    left, right = hip.ln_gdp(tx, *cu(sc, of, wpT, bp, wgT, bg, mask), eps=EPS)
    wl, wr = orf.ln_gdp(x, sc, of, wpT, bp, wgT, bg, mask, EPS)
    check(left, wl, "C4 ln_gdp c=%d %s left" % (c, dt), dt == "bf16")
    check(right, wr, "C4 ln_gdp c=%d %s right" % (c, dt), dt == "bf16")


@pytest.mark.parametrize("dt", TYPES)
@pytest.mark.parametrize("c", WIDTHS)
def test_c4_trimul_epilogue(hip, c, dt):
    rng = rng_for("c4 epi", c, dt)
    x_cm = f32(rng, c, M)
    x, tx = acts(rng, dt == "bf16", M, c)
    ins, ino = f32(rng, c, s=.1, mean=1.), f32(rng, c, s=.1)
    lns, lno = f32(rng, c, s=.1, mean=1.), f32(rng, c, s=.1)
    woT, bo = f16(rng, c, c, s=c ** -.5), f16(rng, c, s=.1)
    wgT, bg = f16(rng, c, c, s=c ** -.5), f16(rng, c, s=.1)
    txcm, tins, tino, tlns, tlno, twoT, tbo, twgT, tbg = cu(x_cm, ins, ino, lns, lno, woT, bo, wgT, bg)
    out = hip.trimul_epilogue(txcm, tx, tins, tino, tlns, tlno, twoT, tbo, twgT, tbg, eps=EPS)
    want = orf.trimul_epilogue(x_cm, x, ins, ino, lns, lno, woT, bo, wgT, bg, None, EPS, False)
    check(out, want, "C4 trimul_epilogue c=%d %s" % (c, dt), dt == "bf16")


@pytest.mark.parametrize("add", (False, True))
@pytest.mark.parametrize("dt", TYPES)
@pytest.mark.parametrize("c,factor", ((64, 2), (64, 4), (128, 4)))
def test_c4_transition(hip, c, factor, dt, add):
    """At c = 64 the resident-weight kernel's 32-row tiles give 8192 tiles over 256 CUs of 16
    waves: every wave runs its second and later tiles (the prefetch of the next rows, issued
    after the stores when add_input reads the rows it overwrites)."""
    rng = rng_for("c4 trans", c, factor, dt, add)
    hd = factor * c
    x, tx = acts(rng, dt == "bf16", M, c)
    sc, of = f32(rng, c, s=.1, mean=1.), f32(rng, c, s=.1)
    w1T, b1 = f16(rng, hd, c, s=c ** -.5), f16(rng, hd, s=.1)
    w2T, b2 = orf.w2_blocked(f16(rng, hd, c, s=hd ** -.5)), f16(rng, c, s=.1)
    out = hip.transition(tx, *cu(sc, of, w1T, b1, w2T, b2), eps=EPS, add_input=add,
                         out=tx if add else None)
    want = orf.transition(x, sc, of, w1T, b1, w2T, b2, None, EPS, add)
    check(out, want, "C4 transition c=%d x%d %s add=%s" % (c, factor, dt, add), dt == "bf16")
