"""Pins the float64 fused-op oracle (oracle/fused.py) against torch's layer_norm, explicit
per-element sums, the transition's blocked weight layout read element by element, closed-form
special cases, a brute-force statement of the keep rule, and the committed golden fixtures.
CPU only.
"""
import os

import numpy as np
import torch

from oracle import fused as orf

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
EPS = 1e-5


def fused_inputs(seed, m=200, c=64):
    """Tiny inputs for every fused op; keep has a computed, a padding, a skipped and a partial
    64-row tile."""
    rng = np.random.default_rng(seed)
    f16 = lambda *s, a=1.0: (rng.standard_normal(s) * a).astype(np.float16).astype(np.float64)
    f32 = lambda *s, a=1.0, mean=0.0: (rng.standard_normal(s) * a + mean).astype(np.float32).astype(np.float64)
    keep = np.ones(m)
    keep[64:128] = 0.0
    keep[128:192] = -1.0
    keep[192:196] = 0.0
    return {
        "x": f16(m, c, a=2.0), "sc": f32(c, a=0.1, mean=1.0), "of": f32(c, a=0.1),
        "wpT": f16(2 * c, c, a=0.1), "bp": f16(2 * c, a=0.1), "wgT": f16(2 * c, c, a=0.1),
        "bg": f16(2 * c, a=0.1), "mask": (rng.random(m) > 0.1).astype(np.float64),
        "x_cm": f32(c, m, a=20.0), "lsc": f32(c, a=0.1, mean=1.0), "lof": f32(c, a=0.1),
        "woT": f16(c, c, a=0.1), "bo": f16(c, a=0.1), "wgT2": f16(c, c, a=0.1), "bg2": f16(c, a=0.1),
        "wT": f16(128, c, a=0.1), "wbT": f16(4, c, a=0.1), "o": f16(m, c), "res": f16(m, c, a=2.0),
        "w1T": f16(4 * c, c, a=c ** -0.5), "b1": f16(4 * c, a=0.1),
        "w2T": orf.w2_blocked(f16(4 * c, c, a=(4 * c) ** -0.5)), "b2": f16(c, a=0.1), "keep": keep,
    }


def test_layer_norm_matches_torch():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((37, 128)) * 3 + 5
    sc, of = rng.standard_normal(128), rng.standard_normal(128)
    want = torch.nn.functional.layer_norm(torch.from_numpy(x), (128,), torch.from_numpy(sc),
                                          torch.from_numpy(of), EPS).numpy()
    np.testing.assert_allclose(orf.layer_norm(x, sc, of, EPS, round_mid=False), want, rtol=1e-12, atol=1e-12)
    # the fp16 rounding point: the rounded LN is the fp16 value of the exact one
    np.testing.assert_array_equal(orf.layer_norm(x, sc, of, EPS), want.astype(np.float16).astype(np.float64))


def test_tile_work_brute_force():
    rng = np.random.default_rng(1)
    for m, rows, other in ((200, 64, -1.0), (200, 64, 0.0), (97, 32, -1.0), (5, 64, 0.0)):
        keep = rng.choice([-1.0, 0.0, 1.0], size=m, p=[0.5, 0.3, 0.2])
        keep[:rows] = -1.0  # one all-negative tile
        got = orf.tile_work(keep, m, rows, other)
        for t, w in enumerate(got):
            vals = [keep[r] if r < m else other for r in range(t * rows, (t + 1) * rows)]
            want = orf.COMPUTE if any(v > 0 for v in vals) else (
                orf.PADDING if any(v == 0 for v in vals) else orf.SKIP)
            assert w == want, (m, rows, other, t)


def test_w2_blocked_layout():
    rng = np.random.default_rng(2)
    w2 = rng.standard_normal((256, 64))
    w2T = orf.w2_blocked(w2)
    for j, c, i in ((0, 0, 0), (3, 63, 63), (1, 17, 5), (2, 40, 33)):
        assert w2T[j, c, i] == w2[64 * j + i, c]
    np.testing.assert_array_equal(orf.w2_unblocked(w2T), w2)


def test_ln_gdp_elements():
    inp = fused_inputs(3)
    left, right = orf.ln_gdp(inp["x"], inp["sc"], inp["of"], inp["wpT"], inp["bp"], inp["wgT"], inp["bg"],
                             np.ones(200), EPS)
    y = orf.layer_norm(inp["x"], inp["sc"], inp["of"], EPS)
    for m, n in ((0, 0), (5, 70), (199, 127), (100, 64)):
        p = sum(y[m, k] * inp["wpT"][n, k] for k in range(64)) + inp["bp"][n]
        g = sum(y[m, k] * inp["wgT"][n, k] for k in range(64)) + inp["bg"][n]
        want = p / (1 + np.exp(-g))
        got = left[n, m] if n < 64 else right[n - 64, m]
        assert abs(got - want) < 1e-12


def test_ln_gdp_mask_rows_and_padding():
    inp = fused_inputs(4)
    mask = np.ones(200)
    mask[:64] = 0.0          # a padding tile: written as zeros
    mask[64:128] = -1.0      # a skipped tile: not written
    mask[130] = -2.0         # inside a computed tile: max(mask, 0) zeroes the row
    left, right = orf.ln_gdp(inp["x"], inp["sc"], inp["of"], inp["wpT"], inp["bp"], inp["wgT"], inp["bg"], mask, EPS)
    assert (left[:, :64] == 0).all() and np.isnan(left[:, 64:128]).all() and (left[:, 130] == 0).all()
    assert np.isfinite(right[:, 128:]).all()


def test_output_projection_explicit():
    inp = fused_inputs(5)
    out = orf.output_projection(inp["o"], inp["woT"], inp["bo"], inp["res"], None)
    for m, n in ((0, 0), (199, 63), (77, 31)):
        want = sum(inp["o"][m, k] * inp["woT"][n, k] for k in range(64)) + inp["bo"][n] + inp["res"][m, n]
        assert abs(out[m, n] - want) < 1e-12


def test_transition_special_cases():
    inp = fused_inputs(6)
    zero2 = np.zeros_like(inp["w2T"])
    out = orf.transition(inp["x"], inp["sc"], inp["of"], inp["w1T"], inp["b1"], zero2, np.zeros(64), None, EPS, True)
    np.testing.assert_array_equal(out, inp["x"])
    zero1 = np.zeros_like(inp["w1T"])
    out = orf.transition(inp["x"], inp["sc"], inp["of"], zero1, np.full(256, -1.0), inp["w2T"], inp["b2"], None, EPS,
                         False)
    np.testing.assert_array_equal(out, np.broadcast_to(inp["b2"], out.shape))


def _torch_ln16(x, sc, of):
    """LayerNorm by torch (float64), rounded to fp16 as the kernels round their GEMM input."""
    y = torch.nn.functional.layer_norm(torch.from_numpy(np.asarray(x, np.float64)), (x.shape[1],),
                                       torch.from_numpy(np.asarray(sc, np.float64)),
                                       torch.from_numpy(np.asarray(of, np.float64)), EPS).numpy()
    return y.astype(np.float16).astype(np.float64)


def test_ln_projection_explicit_sums():
    """p[m, j] = sum_k fp16(LN x)[m, k] wT[j, k] with no bias term, and the head bias
    bias[h, m] = sum_k fp16(LN x)[m, k] wbT[h, k] (cuda/volta_ops.cu:503-541,
    cuda/volta_gdp.h:289-332), from torch's LayerNorm and per-element loops. M, n, heads and K
    all differ, so a transposed or mis-indexed result cannot pass."""
    rng = np.random.default_rng(12)
    m, k, n, heads = 70, 64, 96, 3
    x = (rng.standard_normal((m, k)) * 2 + 0.3).astype(np.float16)
    sc = (1 + 0.2 * rng.standard_normal(k)).astype(np.float32)
    of = (0.2 * rng.standard_normal(k)).astype(np.float32)
    wT = (0.3 * rng.standard_normal((n, k))).astype(np.float16)
    wbT = (0.3 * rng.standard_normal((heads, k))).astype(np.float16)
    p, b = orf.ln_projection(x, sc, of, wT, wbT, None, EPS)
    assert p.shape == (m, n) and b.shape == (heads, m)
    y = _torch_ln16(x, sc, of)
    for mm, j in ((0, 0), (69, 95), (33, 17), (5, 64)):
        want = sum(y[mm, kk] * float(wT[j, kk]) for kk in range(k))
        assert abs(p[mm, j] - want) < 1e-10, (mm, j)
    for h, mm in ((0, 0), (2, 69), (1, 40)):
        want = sum(y[mm, kk] * float(wbT[h, kk]) for kk in range(k))
        assert abs(b[h, mm] - want) < 1e-10, (h, mm)
    # the fp16 rounding of the LN output is observable at this tolerance
    y_exact = torch.nn.functional.layer_norm(torch.from_numpy(x.astype(np.float64)), (k,),
                                             torch.from_numpy(sc.astype(np.float64)),
                                             torch.from_numpy(of.astype(np.float64)), EPS).numpy()
    unrounded = sum(y_exact[69, kk] * float(wT[95, kk]) for kk in range(k))
    assert abs(p[69, 95] - unrounded) > 1e-6


def test_transition_explicit_loop():
    """out[m, c] = sum_j fp16(relu(sum_i fp16(LN x)[m, i] w1[i, j] + b1[j])) w2[j, c] + b2[c]
    (+ x[m, c]) with every weight and bias nonzero (cuda/volta_ops.cu:585-634), the blocked w2T
    built here by its definition w2T[j][c][i] = w2[64 j + i][c] (volta_fused_ffi.h:216-217)."""
    rng = np.random.default_rng(13)
    m, c, hd = 40, 64, 256
    x = (rng.standard_normal((m, c)) * 2).astype(np.float16)
    sc = (1 + 0.2 * rng.standard_normal(c)).astype(np.float32)
    of = (0.2 * rng.standard_normal(c)).astype(np.float32)
    w1 = (rng.standard_normal((c, hd)) * c ** -0.5).astype(np.float16)
    b1 = (0.5 * rng.standard_normal(hd)).astype(np.float16)
    w2 = (rng.standard_normal((hd, c)) * hd ** -0.5).astype(np.float16)
    b2 = (0.5 * rng.standard_normal(c)).astype(np.float16)
    w2T = np.zeros((hd // 64, c, 64), np.float16)
    for j in range(hd // 64):
        for cc in range(c):
            for i in range(64):
                w2T[j, cc, i] = w2[64 * j + i, cc]
    w1T = np.ascontiguousarray(w1.T)
    y = _torch_ln16(x, sc, of)
    for add in (False, True):
        out = orf.transition(x, sc, of, w1T, b1, w2T, b2, None, EPS, add)
        for mm, cc in ((0, 0), (39, 63), (17, 30)):
            hid = [max(sum(y[mm, i] * float(w1[i, j]) for i in range(c)) + float(b1[j]), 0.0)
                   for j in range(hd)]
            hid = np.asarray(hid).astype(np.float16).astype(np.float64)
            want = sum(hid[j] * float(w2[j, cc]) for j in range(hd)) + float(b2[cc])
            if add:
                want += float(x[mm, cc])
            assert abs(out[mm, cc] - want) < 1e-9, (add, mm, cc)


def test_trimul_epilogue_elements():
    inp = fused_inputs(7)
    out = orf.trimul_epilogue(inp["x_cm"], inp["x"], inp["sc"], inp["of"], inp["lsc"], inp["lof"], inp["woT"],
                              inp["bo"], inp["wgT2"], inp["bg2"], None, EPS, True)
    ycol = torch.nn.functional.layer_norm(torch.from_numpy(inp["x_cm"].T.copy()), (64,),
                                          torch.from_numpy(inp["lsc"]), torch.from_numpy(inp["lof"]), EPS).numpy()
    ycol = ycol.astype(np.float16).astype(np.float64)
    a = orf.layer_norm(inp["x"], inp["sc"], inp["of"], EPS)
    for m, o in ((0, 0), (150, 63), (33, 12)):
        lin = sum(ycol[m, c] * inp["woT"][o, c] for c in range(64)) + inp["bo"][o]
        gate = sum(a[m, c] * inp["wgT2"][o, c] for c in range(64)) + inp["bg2"][o]
        want = lin / (1 + np.exp(-gate)) + inp["x"][m, o]
        assert abs(out[m, o] - want) < 1e-9


def test_keep_padding_and_skip():
    inp = fused_inputs(8)
    p, b = orf.ln_projection(inp["x"], inp["sc"], inp["of"], inp["wT"], inp["wbT"], inp["keep"], EPS)
    assert (p[64:128] == 0).all() and np.isnan(p[128:192]).all() and np.isfinite(p[192:]).all()
    assert (b[:, 64:128] == 0).all() and np.isnan(b[:, 128:192]).all()
    t = orf.transition(inp["x"], inp["sc"], inp["of"], inp["w1T"], inp["b1"], inp["w2T"], inp["b2"], inp["keep"],
                       EPS, True)
    assert np.isnan(t[64:192]).all()  # add_input: padding keeps x, which the kernel leaves unwritten


def test_golden_fixtures():
    f = np.load(os.path.join(GOLDEN, "fused_small.npz"))
    inp = fused_inputs(int(f["seed"]))
    l, r = orf.ln_gdp(inp["x"], inp["sc"], inp["of"], inp["wpT"], inp["bp"], inp["wgT"], inp["bg"], inp["mask"], EPS)
    p, b = orf.ln_projection(inp["x"], inp["sc"], inp["of"], inp["wT"], inp["wbT"], inp["keep"], EPS)
    got = {
        "gdp_left": l, "gdp_right": r, "proj_p": p, "proj_bias": b,
        "epi": orf.trimul_epilogue(inp["x_cm"], inp["x"], inp["sc"], inp["of"], inp["lsc"], inp["lof"],
                                   inp["woT"], inp["bo"], inp["wgT2"], inp["bg2"], inp["keep"], EPS, False),
        "outp": orf.output_projection(inp["o"], inp["woT"], inp["bo"], inp["res"], inp["keep"]),
        "trans": orf.transition(inp["x"], inp["sc"], inp["of"], inp["w1T"], inp["b1"], inp["w2T"], inp["b2"],
                                inp["keep"], EPS, True),
    }
    for name, arr in got.items():
        np.testing.assert_allclose(arr, f[name], rtol=1e-12, atol=1e-12, equal_nan=True, err_msg=name)


def test_layer_norm_onepass_matches_torch_and_clamps():
    rng = np.random.default_rng(10)
    x = rng.standard_normal((23, 100)) * 2 + 0.5
    sc, of = rng.standard_normal(100), rng.standard_normal(100)
    want = torch.nn.functional.layer_norm(torch.from_numpy(x), (100,), torch.from_numpy(sc),
                                          torch.from_numpy(of), EPS).numpy()
    np.testing.assert_allclose(orf.layer_norm_onepass(x, sc, of, EPS), want, rtol=1e-9, atol=1e-9)
    # a constant row: E[x^2] - mean^2 is zero (or a rounding below it, clamped), so out = offset
    const = np.full((2, 64), 3.25)
    np.testing.assert_allclose(orf.layer_norm_onepass(const, np.ones(64), of[:64], EPS),
                               np.broadcast_to(of[:64], (2, 64)), atol=1e-12)


def test_gated_dual_proj_elements():
    rng = np.random.default_rng(11)
    M, K, N = 9, 5, 8
    x, wp, wg = rng.standard_normal((M, K)), rng.standard_normal((K, N)), rng.standard_normal((K, N))
    bp, bg, mask = rng.standard_normal(N), rng.standard_normal(N), rng.standard_normal(M)
    for act in (0, 1):
        out = orf.gated_dual_proj(x, wp, bp, wg, bg, mask, act)
        for m, n in ((0, 0), (8, 7), (4, 3)):
            p = sum(x[m, k] * wp[k, n] for k in range(K)) + bp[n]
            g = sum(x[m, k] * wg[k, n] for k in range(K)) + bg[n]
            s = 1.0 / (1.0 + np.exp(-g))
            assert abs(out[m, n] - mask[m] * p * (s if act == 0 else g * s)) < 1e-12
    # a zero mask row zeroes its outputs
    mask[2] = 0.0
    assert np.abs(orf.gated_dual_proj(x, wp, bp, wg, bg, mask, 1)[2]).max() == 0.0
