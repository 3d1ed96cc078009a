"""bf16 activations through the fused entry points on gfx950, against the float64 oracle.

The reference's fused targets are F16 only and its callers decline bf16
(tests/test_fused.py:223-229); this library also takes bf16 activations (x, o, residual and
every activation result bf16 together, weights and biases fp16). A bf16 value is read exactly
into fp32; the LayerNorm output and the transition's hidden activation are rounded to fp16 for
the matrix cores, as on the fp16 path; results are rounded to bf16 once.

The oracle runs on the exact bf16 input values. Tolerance: abs error beyond half a bf16 ulp of
the oracle <= 2e-3 plus 2^-22 of the result's magnitude (the fp32 sum of a residual of large
magnitude before the one rounding), and the reference's rel < 0.02. Cases include inputs of
magnitude 1e5, beyond fp16's range, which bf16 callers can hold.
"""
import zlib

import numpy as np
import pytest
import torch

from conftest import abs_excess, rel
from oracle import fused as orf

pytestmark = pytest.mark.gpu

ATOL = 2e-3
REL = 0.02
EPS = 1e-5
ROWS = (59, 4101, 67600)


def rng_for(*key):
    return np.random.default_rng(zlib.crc32(repr(key).encode()))


def bf(rng, *shape, s=0.5, mean=0.0):
    """float64 values exactly representable in bf16, and the bf16 tensor on the GPU."""
    t = torch.from_numpy(rng.standard_normal(shape) * s + mean).to(torch.bfloat16)
    return t.double().numpy(), t.cuda()


def f16(rng, *shape, s=0.5, mean=0.0):
    return (rng.standard_normal(shape) * s + mean).astype(np.float16)


def f32(rng, *shape, s=0.5, mean=0.0):
    return (rng.standard_normal(shape) * s + mean).astype(np.float32)


def cu(*xs):
    return [torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in xs]


def npy(t):
    torch.cuda.synchronize()
    assert t.dtype == torch.bfloat16
    return t.double().cpu().numpy()


def check(got, want, label):
    tol = ATOL + 2.0 ** -22 * float(np.nanmax(np.abs(want), initial=0.0))
    e = abs_excess(got, want, bf16_out=True)
    r = rel(got, want)
    assert e <= tol and r < REL, "%s: abs excess %.2e (tol %.1e), rel %.2e" % (label, e, tol, r)


AMPS = ((2.0, 0.0), (3e4, 1e5))  # (spread, mean) of the LayerNorm inputs


@pytest.mark.parametrize("a,ci", ((128, 128), (64, 64), (128, 64)))
@pytest.mark.parametrize("m", ROWS)
@pytest.mark.parametrize("s,mean", AMPS)
def test_ln_gdp_bf16(hip, a, ci, m, s, mean):
    rng = rng_for("gdp bf16", a, ci, m, mean)
    x, tx = bf(rng, m, a, s=s, mean=mean)
    mask = (rng.uniform(size=m) > .1).astype(np.float16)
    sc, of = f32(rng, a, s=.1, mean=1.), f32(rng, a, s=.1)
    wpT, wgT = f16(rng, 2 * ci, a, s=.1), f16(rng, 2 * ci, a, s=.1)
    bp, bg = f16(rng, 2 * ci, s=.1), f16(rng, 2 * ci, s=.1)
    left, right = hip.ln_gdp(tx, *cu(sc, of, wpT, bp, wgT, bg, mask), eps=EPS)
    wl, wr = orf.ln_gdp(x, sc, of, wpT, bp, wgT, bg, mask, EPS)
    check(npy(left), wl, "left")
    check(npy(right), wr, "right")


@pytest.mark.parametrize("a,ci", ((128, 128), (64, 64), (128, 64)))
@pytest.mark.parametrize("m", ROWS)
@pytest.mark.parametrize("s,mean", AMPS)
@pytest.mark.parametrize("add", (False, True))
def test_trimul_epilogue_bf16(hip, a, ci, m, s, mean, add):
    rng = rng_for("epi bf16", a, ci, m, mean, add)
    x, tx = bf(rng, m, a, s=s, mean=mean)
    sc, of = f32(rng, a, s=.1, mean=1.), f32(rng, a, s=.1)
    x_cm = f32(rng, ci, m, s=50.)
    lsc, lof = f32(rng, ci, s=.1, mean=1.), f32(rng, ci, s=.1)
    woT, bo = f16(rng, a, ci, s=.1), f16(rng, a, s=.1)
    wgT, bg = f16(rng, a, a, s=.1), f16(rng, a, s=.1)
    t = cu(x_cm, sc, of, lsc, lof, woT, bo, wgT, bg)
    out = hip.trimul_epilogue(t[0], tx, *t[1:], eps=EPS, add_input=add)
    want = orf.trimul_epilogue(x_cm, x, sc, of, lsc, lof, woT, bo, wgT, bg, None, EPS, add)
    check(npy(out), want, "epilogue")


@pytest.mark.parametrize("a,n", ((128, 128), (64, 64), (64, 128)))
@pytest.mark.parametrize("m", ROWS)
@pytest.mark.parametrize("slots,heads", ((4, 4), (0, 8)))
def test_ln_projection_bf16(hip, a, n, m, slots, heads):
    rng = rng_for("proj bf16", a, n, m, slots, heads)
    x, tx = bf(rng, m, a, s=2.)
    sc, of = f32(rng, a, s=.1, mean=1.), f32(rng, a, s=.1)
    w = f16(rng, slots, a, n, s=.1)
    wT = np.ascontiguousarray(w.transpose(0, 2, 1).reshape(slots * n, a)) if slots else None
    wbT = f16(rng, heads, a, s=.1)
    tsc, tof, twb = cu(sc, of, wbT)
    twT = cu(wT)[0] if slots else None
    p, b = hip.ln_projection(tx, tsc, tof, twT, twb, eps=EPS)
    wp, wb = orf.ln_projection(x, sc, of, wT, wbT, None, EPS)
    if slots:
        check(npy(p), wp, "p")
    check(npy(b), wb, "bias")


@pytest.mark.parametrize("k,c", ((128, 128), (64, 64), (128, 64), (64, 128)))
@pytest.mark.parametrize("m", ROWS)
@pytest.mark.parametrize("residual", (True, False))
def test_output_projection_bf16(hip, k, c, m, residual):
    # o enters the matrix cores as fp16: exact for attention outputs of fp16 range
    rng = rng_for("out bf16", k, c, m, residual)
    o, to = bf(rng, m, k)
    wT, b = f16(rng, c, k, s=.1), f16(rng, c, s=.1)
    r, tr = bf(rng, m, c, s=3e4, mean=1e5) if residual else (None, None)
    tw, tb = cu(wT, b)
    out = hip.output_projection(to, tw, tb, tr)
    check(npy(out), orf.output_projection(o, wT, b, r, None), "out")


@pytest.mark.parametrize("c,factor", ((128, 4), (64, 2), (256, 4)))
@pytest.mark.parametrize("m", ROWS)
@pytest.mark.parametrize("s,mean", AMPS)
@pytest.mark.parametrize("add", (False, True))
def test_transition_bf16(hip, c, factor, m, s, mean, add):
    rng = rng_for("trans bf16", c, factor, m, mean, add)
    hd = factor * c
    x, tx = bf(rng, m, c, s=s, mean=mean)
    sc, of = f32(rng, c, s=.1, mean=1.), f32(rng, c, s=.1)
    w1T = np.ascontiguousarray(f16(rng, c, hd, s=c ** -.5).T)
    b1 = f16(rng, hd, s=.1)
    w2T = orf.w2_blocked(f16(rng, hd, c, s=hd ** -.5))
    b2 = f16(rng, c, s=.1)
    out = hip.transition(tx, *cu(sc, of, w1T, b1, w2T, b2), eps=EPS, add_input=add)
    want = orf.transition(x, sc, of, w1T, b1, w2T, b2, None, EPS, add)
    check(npy(out), want, "transition")


@pytest.mark.parametrize("c", (64, 128))
def test_keep_bf16(hip, c):
    """keep with bf16 activations: real rows identical with and without keep, rows of padded
    tiles zero or (where the output aliases x) unchanged (tests/test_keep.py); the transition at
    4C (and 2C at c = 64) and the tri-mul epilogue."""
    S, n = 192, 65
    live = ((np.arange(S) < n)[:, None] & (np.arange(S) < n)[None, :]).reshape(-1)
    rng = rng_for("keep bf16", c)
    m = live.size
    x, tx = bf(rng, m, c, s=2.)
    tkeep = cu(live.astype(np.float16))[0]
    sc, of = f32(rng, c, s=.1, mean=1.), f32(rng, c, s=.1)

    def check_rows(kept, plain, pad, label):
        assert np.array_equal(kept[live], plain[live]), "real rows differ (%s)" % label
        # padding is decided per row tile: a padded row is the plain result (its tile holds a
        # live row) or the padding value (x where the output aliases it, else zero)
        ok = (kept[~live] == plain[~live]) | (kept[~live] == pad)
        assert ok.all(), "padded rows (%s)" % label
        assert (kept[~live] == pad).any(), "no row was padded (%s)" % label

    for factor in ((2, 4) if c == 64 else (4,)):
        hd = factor * c
        tw = cu(sc, of, np.ascontiguousarray(f16(rng, c, hd, s=c ** -.5).T), f16(rng, hd, s=.1),
                orf.w2_blocked(f16(rng, hd, c, s=hd ** -.5)), f16(rng, c, s=.1))
        for add in (False, True):
            a0, a1 = tx.clone(), tx.clone()
            plain = npy(hip.transition(a0, *tw, eps=EPS, add_input=add, out=a0 if add else None))
            kept = npy(hip.transition(a1, *tw, keep=tkeep, eps=EPS, add_input=add,
                                      out=a1 if add else None))
            check_rows(kept, plain, x[~live] if add else 0.0,
                       "transition c=%d x%d add=%s" % (c, factor, add))
    x_cm = f32(rng, c, m, s=20.)
    g = cu(x_cm, sc, of, f32(rng, c, s=.1, mean=1.), f32(rng, c, s=.1), f16(rng, c, c, s=.1),
           f16(rng, c, s=.1), f16(rng, c, c, s=.1), f16(rng, c, s=.1))
    for add in (False, True):
        a0, a1 = tx.clone(), tx.clone()
        plain = npy(hip.trimul_epilogue(g[0], a0, *g[1:], eps=EPS, add_input=add,
                                        out=a0 if add else None))
        kept = npy(hip.trimul_epilogue(g[0], a1, *g[1:], keep=tkeep, eps=EPS, add_input=add,
                                       out=a1 if add else None))
        check_rows(kept, plain, x[~live] if add else 0.0, "epilogue c=%d add=%s" % (c, add))
