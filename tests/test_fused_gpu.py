"""The LayerNorm-fused projections on gfx950 against the float64 oracle, through the C ABI.

Cases follow the reference's tests/test_fused.py (row counts 1, 59, 4101 and a 260 x 260 pair,
widths (128,128), (64,64), (128,64), the epilogue's x_cm at amplitude 50 and at mean 1e3, slot
and head counts (4,4), (3,8) and bias-only, output projections with and without a residual,
transitions (128,x4), (64,x2), (64,x4), (256,x4)) and tests/test_keep.py (real rows identical
with and without keep; padded rows zero or, where the output aliases its input, unchanged;
keep < 0 rows never written).

Tolerance (fp16 I/O): abs error beyond half an fp16 ulp of the oracle <= 2e-3, with the oracle
rounding the LayerNorm output and the hidden activation to fp16 where the kernels do; the
reference's own metric rel < 0.02 is checked as well.
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
WIDTHS = ((128, 128), (64, 64), (128, 64))


def rng_for(*key):
    return np.random.default_rng(zlib.crc32(repr(key).encode()))


def f16(rng, *shape, s=0.5, mean=0.0):
    return (rng.standard_normal(shape) * s + mean).astype(np.float16)


def f32(rng, *shape, s=0.5, mean=0.0):
    return (rng.standard_normal(shape) * s + mean).astype(np.float32)


def cu(*xs):
    return [torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in xs]


def npy(t):
    torch.cuda.synchronize()
    return t.float().cpu().numpy()


def check(got, want, label, tol=ATOL):
    e = abs_excess(got, want)
    r = rel(got, want)
    assert e <= tol and r < REL, "%s: abs excess %.2e (tol %.0e), rel %.2e" % (label, e, tol, r)


ROWS = (1, 59, 4101, 260 * 260)


@pytest.mark.parametrize("a,ci", WIDTHS)
@pytest.mark.parametrize("m", ROWS)
def test_ln_gdp(hip, a, ci, m):
    rng = rng_for("gdp", a, ci, m)
    x = f16(rng, m, a, s=2.)
    mask = (rng.uniform(size=m) > .1).astype(np.float16)
    sc, of = f32(rng, a, s=.1, mean=1.), f32(rng, a, s=.1)
    wpT, wgT = f16(rng, 2 * ci, a, s=.1), f16(rng, 2 * ci, a, s=.1)
    bp, bg = f16(rng, 2 * ci, s=.1), f16(rng, 2 * ci, s=.1)
    left, right = hip.ln_gdp(*cu(x, sc, of, wpT, bp, wgT, bg, mask), eps=EPS)
    wl, wr = orf.ln_gdp(x, sc, of, wpT, bp, wgT, bg, mask, EPS)
    check(npy(left), wl, "left")
    check(npy(right), wr, "right")


@pytest.mark.parametrize("a,ci", WIDTHS)
@pytest.mark.parametrize("m", ROWS)  # 260 x 260: more 32-row tiles than workgroups
@pytest.mark.parametrize("amp,mean", ((50., 0.), (5., 1e3)))
@pytest.mark.parametrize("add", (False, True))
def test_trimul_epilogue(hip, a, ci, m, amp, mean, add):
    rng = rng_for("epi", a, ci, m, amp, add)
    x = f16(rng, m, a, s=2.)
    sc, of = f32(rng, a, s=.1, mean=1.), f32(rng, a, s=.1)
    x_cm = f32(rng, ci, m, s=amp, mean=mean)
    lsc, lof = f32(rng, ci, s=.1, mean=1.), f32(rng, ci, s=.1)
    woT, bo = f16(rng, a, ci, s=.1), f16(rng, a, s=.1)
    wgT, bg = f16(rng, a, a, s=.1), f16(rng, a, s=.1)
    args = cu(x_cm, x, sc, of, lsc, lof, woT, bo, wgT, bg)
    out = hip.trimul_epilogue(*args, eps=EPS, add_input=add)
    want = orf.trimul_epilogue(x_cm, x, sc, of, lsc, lof, woT, bo, wgT, bg, None, EPS, add)
    check(npy(out), want, "epilogue")


@pytest.mark.parametrize("a,n", WIDTHS + ((64, 128),))  # (64, 128) with 4 slots: the C4 c = 64 shape
@pytest.mark.parametrize("m", ROWS)
@pytest.mark.parametrize("slots,heads", ((4, 4), (3, 8), (0, 8)))
def test_ln_projection(hip, a, n, m, slots, heads):
    # at 260 x 260 rows every workgroup runs several tiles (its rotated next-tile prefetch)
    rng = rng_for("proj", a, n, m, slots, heads)
    x = f16(rng, m, a, s=2.)
    sc, of = f32(rng, a, s=.1, mean=1.), f32(rng, a, s=.1)
    w = f16(rng, slots, a, n, s=.1)
    # the wrapper's re-layout: w [slots, a, n] -> wT [slots n, a], slot major
    wT = np.ascontiguousarray(w.transpose(0, 2, 1).reshape(slots * n, a)) if slots else None
    wbT = f16(rng, heads, a, s=.1)
    tx, tsc, tof, twb = cu(x, sc, of, wbT)
    twT = cu(wT)[0] if slots else None
    p, b = hip.ln_projection(tx, tsc, tof, twT, twb, eps=EPS)
    wp, wb = orf.ln_projection(x, sc, of, wT, wbT, None, EPS)
    if slots:
        check(npy(p), wp, "p")
    check(npy(b), wb, "bias")


@pytest.mark.parametrize("k,c", ((128, 128), (64, 64), (128, 64), (64, 128)))
@pytest.mark.parametrize("m", ROWS)
@pytest.mark.parametrize("residual", (True, False))
def test_output_projection(hip, k, c, m, residual):
    rng = rng_for("out", k, c, m, residual)
    o, wT, b = f16(rng, m, k), f16(rng, c, k, s=.1), f16(rng, c, s=.1)
    r = f16(rng, m, c, s=2.) if residual else None
    to, tw, tb = cu(o, wT, b)
    tr = cu(r)[0] if residual else None
    out = hip.output_projection(to, tw, tb, tr)
    check(npy(out), orf.output_projection(o, wT, b, r, None), "out")


@pytest.mark.parametrize("c,factor", ((128, 4), (64, 2), (64, 4), (256, 4)))
@pytest.mark.parametrize("m", ROWS)
@pytest.mark.parametrize("add", (False, True))
def test_transition(hip, c, factor, m, add):
    rng = rng_for("trans", c, factor, m, add)
    hd = factor * c
    x = f16(rng, m, c, s=2.)
    sc, of = f32(rng, c, s=.1, mean=1.), f32(rng, c, s=.1)
    w1 = f16(rng, c, hd, s=c ** -.5)
    b1 = f16(rng, hd, s=.1)
    w2 = f16(rng, hd, c, s=hd ** -.5)
    b2 = f16(rng, c, s=.1)
    w1T = np.ascontiguousarray(w1.T)
    w2T = orf.w2_blocked(w2)
    out = hip.transition(*cu(x, sc, of, w1T, b1, w2T, b2), eps=EPS, add_input=add)
    want = orf.transition(x, sc, of, w1T, b1, w2T, b2, None, EPS, add)
    check(npy(out), want, "transition")


# ---- keep (tests/test_keep.py) ---------------------------------------------------------------

def pair_keep(S, n):
    live = np.arange(S) < n
    return (live[:, None] & live[None, :]).reshape(-1)


KEEP_CASES = [("pair S=256 n=200", pair_keep(256, 200)), ("pair S=192 n=65", pair_keep(192, 65)),
              ("msa X=508 Y=200 live=37",
               np.broadcast_to((np.arange(508) < 37)[:, None], (508, 200)).reshape(-1))]


def check_keep(got_keep, got_plain, keep_rows, pad_value, label, rows_axis=0):
    """Real rows identical; padded rows identical to the plain call or pad_value; finite."""
    g, b = np.asarray(got_keep), np.asarray(got_plain)
    if rows_axis == 1:
        g, b = g.T, b.T
    k = keep_rows.astype(bool)
    assert np.isfinite(g).all(), label + ": non-finite"
    assert np.array_equal(g[k], b[k]), label + ": real rows differ from the call without keep"
    pv = np.broadcast_to(pad_value, g.shape)[~k] if np.ndim(pad_value) else pad_value
    pad_ok = (g[~k] == b[~k]) | (g[~k] == pv)
    assert pad_ok.all(), label + ": a padded row is neither the plain result nor the padding value"


@pytest.mark.parametrize("c", (64, 128))
@pytest.mark.parametrize("label,live", KEEP_CASES, ids=[c[0] for c in KEEP_CASES])
def test_keep(hip, label, live, c):
    """At c = 64 the transition (2C and 4C) runs the resident-weight kernel, whose keep decision
    is a ballot per 64-row unit, and the epilogue its C = 64 tiles; at c = 128 the chunked
    transition and the 128-channel epilogue."""
    rng = rng_for("keep", label, c)
    m, n, h = live.size, 128, 4
    keep = live.astype(np.float16)
    tkeep = cu(keep)[0]
    x = f16(rng, m, c, s=2.)
    sc, of = f32(rng, c, s=.1, mean=1.), f32(rng, c, s=.1)
    tx, tsc, tof = cu(x, sc, of)
    # transition, with and without add_input
    for factor in ((2, 4) if c == 64 else (4,)):
        hd = factor * c
        w1T, b1 = f16(rng, hd, c, s=c ** -.5), f16(rng, hd, s=.1)
        w2T, b2 = orf.w2_blocked(f16(rng, hd, c, s=hd ** -.5)), f16(rng, c, s=.1)
        tw = cu(w1T, b1, w2T, b2)
        for add in (False, True):
            plain_in = tx.clone()
            plain = npy(hip.transition(plain_in, tsc, tof, *tw, eps=EPS, add_input=add,
                                       out=plain_in if add else None))
            kin = tx.clone()
            kept = npy(hip.transition(kin, tsc, tof, *tw, keep=tkeep, eps=EPS, add_input=add,
                                      out=kin if add else None))
            check_keep(kept, plain, live, x.astype(np.float32) if add else 0.0,
                       "%s transition c=%d x%d add=%s" % (label, c, factor, add))
    # ln_projection
    wT, wbT = f16(rng, 4 * n, c, s=.1), f16(rng, h, c, s=.1)
    twT, twb = cu(wT, wbT)
    p0, b0 = (npy(t) for t in hip.ln_projection(tx, tsc, tof, twT, twb, eps=EPS))
    p1, b1_ = (npy(t) for t in hip.ln_projection(tx, tsc, tof, twT, twb, keep=tkeep, eps=EPS))
    check_keep(p1, p0, live, 0.0, label + " ln_projection p")
    check_keep(b1_, b0, live, 0.0, label + " ln_projection bias", rows_axis=1)
    # output_projection with and without a residual
    o, woT, bo = f16(rng, m, n), f16(rng, c, n, s=.1), f16(rng, c, s=.1)
    to, two, tbo = cu(o, woT, bo)
    for with_res in (True, False):
        res0 = tx.clone()
        plain = npy(hip.output_projection(to, two, tbo, res0 if with_res else None,
                                          out=res0 if with_res else None))
        res1 = tx.clone()
        kept = npy(hip.output_projection(to, two, tbo, res1 if with_res else None, keep=tkeep,
                                         out=res1 if with_res else None))
        check_keep(kept, plain, live, x.astype(np.float32) if with_res else 0.0,
                   "%s output_projection residual=%s" % (label, with_res))
    if label.startswith("pair"):
        # trimul epilogue, and ln_gdp whose mask is its keep: padded columns exactly zero
        tri = f32(rng, c, m, s=20.)
        g = (f32(rng, c, s=.1, mean=1.), f32(rng, c, s=.1), f16(rng, c, c, s=.1), f16(rng, c, s=.1),
             f16(rng, c, c, s=.1), f16(rng, c, s=.1))
        tg = cu(tri, *g)
        for add in (False, True):
            x0 = tx.clone()
            plain = npy(hip.trimul_epilogue(tg[0], x0, tsc, tof, *tg[1:], eps=EPS, add_input=add,
                                            out=x0 if add else None))
            x1 = tx.clone()
            kept = npy(hip.trimul_epilogue(tg[0], x1, tsc, tof, *tg[1:], keep=tkeep, eps=EPS,
                                           add_input=add, out=x1 if add else None))
            check_keep(kept, plain, live, x.astype(np.float32) if add else 0.0,
                       "%s epilogue add=%s" % (label, add))
        gw = (f16(rng, 2 * c, c, s=.1), f16(rng, 2 * c, s=.1), f16(rng, 2 * c, c, s=.1),
              f16(rng, 2 * c, s=.1))
        left, right = hip.ln_gdp(tx, tsc, tof, *cu(*gw), tkeep, eps=EPS)
        wl, wr = orf.ln_gdp(x, sc, of, *gw, keep, EPS)
        for got, want in ((npy(left), wl), (npy(right), wr)):
            check(got[:, live], want[:, live], label + " ln_gdp live")
            assert np.abs(got[:, ~live]).max(initial=0) == 0, label + " ln_gdp padding not zero"


def test_keep_below_zero_writes_nothing(hip):
    """keep < 0 past the live block (rounded to 128): nothing is written there
    (tests/test_keep.py:217-251)."""
    S, n = 256, 200
    R = -(-n // 128) * 128
    tok, ins = np.arange(S) < n, np.arange(S) < R
    mask = (tok[:, None] & tok[None, :]).astype(np.float16)
    region = np.where(ins[:, None] & ins[None, :], mask, -1).astype(np.float16).reshape(-1)
    outside = ~(ins[:, None] & ins[None, :]).reshape(-1)
    rng = rng_for("below")
    c = 128
    x = f16(rng, S * S, c, s=2.)
    sc, of = f32(rng, c, s=.1, mean=1.), f32(rng, c, s=.1)
    wT, wbT = f16(rng, 4 * 128, c, s=.1), f16(rng, 4, c, s=.1)
    tx, tsc, tof, twT, twb, treg = cu(x, sc, of, wT, wbT, region)
    p = torch.full((S * S, 512), 7.0, dtype=torch.float16, device="cuda")
    b = torch.full((4, S * S), 7.0, dtype=torch.float16, device="cuda")
    # write into sentinel-filled results: rows with keep < 0 must keep the sentinel
    from colabfold_legacy_kernels import hip as h
    bufs = [h.buffer(t) for t in (tx, tsc, tof, twT, twb, treg, p, b)]
    h._check(h.lib().clk_ln_projection(h._stream(tx), *map(h._ref, bufs), EPS, 512, 4, 1))
    pn, bn = npy(p), npy(b)
    assert (pn[outside] == 7.0).all() and (bn[:, outside] == 7.0).all()
    live = mask.reshape(-1) > 0
    wp, wb = orf.ln_projection(x, sc, of, wT, wbT, None, EPS)
    check(pn[live], wp[live], "live p")
    check(bn[:, live], wb[:, live], "live bias")


@pytest.mark.parametrize("a,ci", WIDTHS + ((64, 128),))
@pytest.mark.parametrize("m", (421, 424, 4096))
def test_ln_gdp_keep_rule_per_tile(hip, a, ci, m):
    """ln_gdp's mask is its keep, decided per 64-row tile (cuda/volta_gdp.h:114-136): a tile with
    a row above zero is computed, one with all rows at most zero and one at zero is padded with
    zeros, and any other tile (all below zero, or NaN) is not written. Rows counts divisible by 8
    take the 16-byte store path; 424 ends in a 40-row tile whose third 16-row group has 8 rows.
    The results start as a sentinel, so unwritten columns must still hold it."""
    rng = rng_for("gdp keep", a, ci, m)
    x = f16(rng, m, a, s=2.)
    sc, of = f32(rng, a, s=.1, mean=1.), f32(rng, a, s=.1)
    wpT, wgT = f16(rng, 2 * ci, a, s=.1), f16(rng, 2 * ci, a, s=.1)
    bp, bg = f16(rng, 2 * ci, s=.1), f16(rng, 2 * ci, s=.1)
    mask = (rng.uniform(size=m) > .2).astype(np.float16)
    mask[rng.uniform(size=m) < .1] = -1
    tiles = -(-m // 64)
    kinds = ["compute", "padding", "skip", "padding_mixed", "one_live", "nan", "skip"]
    for t in range(tiles - 1):
        rows = slice(64 * t, 64 * t + 64)
        kind = kinds[t % len(kinds)]
        if kind == "padding":
            mask[rows] = 0
        elif kind == "skip":
            mask[rows] = -1
        elif kind == "padding_mixed":
            mask[rows] = np.where(rng.uniform(size=64) < .5, 0, -1)
        elif kind == "one_live":
            mask[rows] = -1
            mask[64 * t + 17] = 0.5
        elif kind == "nan":
            mask[rows] = np.nan
    tx, tsc, tof, twp, tbp, twg, tbg, tmask = cu(x, sc, of, wpT, bp, wgT, bg, mask)
    left = torch.full((ci, m), 7.0, dtype=torch.float16, device="cuda")
    right = torch.full((ci, m), 7.0, dtype=torch.float16, device="cuda")
    from colabfold_legacy_kernels import hip as h
    bufs = [h.buffer(t) for t in (tx, tsc, tof, twp, tbp, twg, tbg, tmask, left, right)]
    h._check(h.lib().clk_ln_gdp(h._stream(tx), *map(h._ref, bufs), EPS))
    wl, wr = orf.ln_gdp(x, sc, of, wpT, bp, wgT, bg, mask, EPS)
    for got, want, label in ((npy(left), wl, "left"), (npy(right), wr, "right")):
        unwritten = np.isnan(want)
        assert unwritten.any() == ("skip" in kinds[:tiles - 1]), label
        assert (got[unwritten] == 7.0).all(), label + ": a skipped tile was written"
        check(got[~unwritten], want[~unwritten], label)
        padded = np.zeros(want.shape, bool)
        for t in range(tiles - 1):
            if kinds[t % len(kinds)] in ("padding", "padding_mixed"):
                padded[:, 64 * t:64 * t + 64] = True
        assert (got[padded] == 0).all() and not np.signbit(got[padded]).any(), label + ": padding not +0"


@pytest.mark.parametrize("a,ci", WIDTHS + ((64, 128),))
def test_ln_gdp_layer_norm_parameters_of_each_call(hip, a, ci):
    """Consecutive calls with different LayerNorm scale and offset: each call's first tiles must
    use its own parameters, not what an earlier call left in LDS (the parameters are staged in
    LDS at the start of the kernel and read by every wave)."""
    m = 67600  # divisible by 8: the 16-byte store path, with more tiles than workgroups
    rng = rng_for("gdp params", a, ci)
    x = f16(rng, m, a, s=2.)
    wpT, wgT = f16(rng, 2 * ci, a, s=.1), f16(rng, 2 * ci, a, s=.1)
    bp, bg = f16(rng, 2 * ci, s=.1), f16(rng, 2 * ci, s=.1)
    mask = (rng.uniform(size=m) > .1).astype(np.float16)
    tx, twp, tbp, twg, tbg, tmask = cu(x, wpT, bp, wgT, bg, mask)
    for call in range(3):
        sc, of = f32(rng, a, s=.1, mean=1.), f32(rng, a, s=.1)  # fresh draws each call
        tsc, tof = cu(sc, of)
        left, right = hip.ln_gdp(tx, tsc, tof, twp, tbp, twg, tbg, tmask, eps=EPS)
        wl, wr = orf.ln_gdp(x, sc, of, wpT, bp, wgT, bg, mask, EPS)
        check(npy(left), wl, "call %d left" % call)
        check(npy(right), wr, "call %d right" % call)
