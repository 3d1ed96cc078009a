"""The caller glue on gfx950: attention as a differentiable torch op (the custom_vjp wiring of
tests/test_attn_bwd.py:262-281) against the float64 oracle's gradients, the gate's gradient,
and the fused ops called with natural weight shapes, which must agree bit for bit with the C ABI
called on explicitly re-laid-out weights and with the oracle."""
import numpy as np
import pytest
import torch

from colabfold_legacy_kernels import layouts, torch_ops
from conftest import abs_excess, record_error
from oracle import attention as ora
from oracle import fused as orf
from test_attention_gpu import GRAD_ATOL, OUT_ATOL, REL_TOL, check, dev, host, inputs

pytestmark = pytest.mark.gpu


def test_autograd_attention(hip):
    n, h, s, d = 3, 4, 96, 32
    q, k, v, bias, km, dout = inputs(n, h, s, s, d, 21)
    tq, tk, tv, tb = (t.requires_grad_() for t in dev(q, k, v, bias))
    tm, tdo = dev(km, dout)
    out = torch_ops.attention(tq, tk, tv, tb, tm)
    (out.float() * tdo.float()).sum().backward()
    assert tb.grad.dtype == torch.float16, "dbias is cast to the bias dtype"
    got = dict(zip(("out", "dq", "dk", "dv", "dbias"),
                   host(out.detach(), tq.grad, tk.grad, tv.grad, tb.grad)))
    ref = dict(zip(("dq", "dk", "dv", "dbias"), ora.attention_bwd(q, k, v, bias, km, dout, d ** -0.5)))
    ref["out"] = ora.attention_fwd(q, k, v, bias, km, d ** -0.5)[0]
    # dbias went through an fp16 cast here, so it is judged as an fp16 result
    got["dbias"] = got["dbias"].astype(np.float16)
    check(got, ref, "autograd", names=("out", "dq", "dk", "dv"))
    raw, e, r = record_error("autograd", "dbias", got["dbias"], ref["dbias"], fp16_out=True)
    assert e <= GRAD_ATOL and r < REL_TOL, (raw, e, r)


def test_autograd_without_bias_grad(hip):
    """A bias that needs no gradient runs the backward without want_dbias; dq, dk, dv are the
    same bits as with it."""
    q, k, v, bias, km, dout = inputs(2, 2, 64, 80, 32, 22)
    grads = []
    for need_bias in (True, False):
        tq, tk, tv = (t.requires_grad_() for t in dev(q, k, v))
        tb = dev(bias)[0].requires_grad_(need_bias)
        tm, tdo = dev(km, dout)
        out = torch_ops.attention(tq, tk, tv, tb, tm)
        out.backward(tdo)
        grads.append(host(tq.grad, tk.grad, tv.grad))
        assert (tb.grad is None) != need_bias
    for x, y in zip(*grads):
        assert np.array_equal(x, y)


def test_gated_attention_gate_gradient(hip):
    """d/dg sum(o sigmoid(g + gb) dout) = o s (1 - s) dout, with o the oracle's attention."""
    n, h, s, d = 2, 2, 64, 32
    q, k, v, bias, km, dout = inputs(n, h, s, s, d, 23)
    rng = np.random.default_rng(24)
    gate = rng.standard_normal((n, h, s, d)).astype(np.float16)
    gb = (0.3 * rng.standard_normal((h, d))).astype(np.float16)
    tq, tk, tv, tb, tm, tdo, tgb = dev(q, k, v, bias, km, dout, gb)
    tg = dev(gate)[0].requires_grad_()
    out = torch_ops.gated_attention(tq, tk, tv, tb, tm, tg, tgb)
    out.backward(tdo)
    o = ora.attention_fwd(q, k, v, bias, km, d ** -0.5)[0]
    sg = 1.0 / (1.0 + np.exp(-(gate.astype(np.float64) + gb.astype(np.float64)[None, :, None, :])))
    want_out = o * sg
    want_dg = o * sg * (1 - sg) * dout.astype(np.float64)
    got_out, got_dg = host(out.detach(), tg.grad)
    check({"out": got_out, "dg": got_dg}, {"out": want_out, "dg": want_dg}, "gated", names=("out",))
    raw, e, r = record_error("gated", "dgate", got_dg, want_dg)
    assert e <= GRAD_ATOL and r < REL_TOL, (raw, e, r)


def test_packed_trim_with_glue_limits(hip):
    """trim_limits on the device feeds VoltaMmaPackedTrim (tests/test_packed_attention.py:53-57),
    judged as the reference judges trim (76-85): queries below the largest limit as the oracle,
    the rest of a live row either the untrimmed result or zero, a row with no live key zero."""
    rng = np.random.default_rng(25)
    x, y, hh, d = 12, 150, 4, 32
    p = (rng.standard_normal((x, y, 4, hh, d)) * 0.5).astype(np.float16)
    bias = (rng.standard_normal((hh, y, y)) * 0.5).astype(np.float16)
    km = np.zeros((x, y), np.uint8)
    for r in range(x):
        km[r, :rng.integers(0, y + 1)] = 1
    km[3] = 0
    gb = np.zeros((hh, d), np.float16)
    tp, tb, tm, tg = dev(p, bias, km, gb)
    lims = torch_ops.trim_limits(tm)
    assert lims.tolist() == ora.trim_limits(km).tolist()
    t, o = host(hip.attention_packed(tp, tb, tm, tg, d ** -0.5, lims=lims),
                hip.attention_packed(tp, tb, tm, tg, d ** -0.5))
    want = ora.attention_packed(p, bias, km, gb, False)
    top = int(lims[-1])
    alive = km.any(axis=1)
    check({"out": t[alive][:, :top]}, {"out": want[alive][:, :top]}, "trim glue", names=("out",))
    pad, full = t[alive][:, top:], o[alive][:, top:]
    assert ((pad == full) | (pad == 0)).all(), "padded queries neither the untrimmed value nor zero"
    assert (t[~alive] == 0).all(), "a row with no live key was written"


def f16(rng, *shape, s=0.5):
    return (rng.standard_normal(shape) * s).astype(np.float16)


def f32(rng, *shape, s=0.1, mean=0.0):
    return (rng.standard_normal(shape) * s + mean).astype(np.float32)


def test_fused_natural_layouts(hip):
    rng = np.random.default_rng(26)
    m, a, ci = 4101, 128, 64
    x = f16(rng, m, a, s=2.0)
    sc, of = f32(rng, a, mean=1.0), f32(rng, a)
    tx, tsc, tof = dev(x, sc, of)
    # ln_gated_dual_proj: wp, wg [a, 2 ci]
    wp, wg, bp, bg = f16(rng, a, 2 * ci, s=.1), f16(rng, a, 2 * ci, s=.1), f16(rng, 2 * ci, s=.1), f16(rng, 2 * ci, s=.1)
    mask = (rng.random(m) > 0.1).astype(np.float16)
    twp, twg, tbp, tbg, tmask = dev(wp, wg, bp, bg, mask)
    left, right = torch_ops.ln_gated_dual_proj(tx, tsc, tof, twp, tbp, twg, tbg, tmask)
    l2, r2 = hip.ln_gdp(tx, tsc, tof, twp.t().contiguous(), tbp, twg.t().contiguous(), tbg, tmask)
    assert torch.equal(left, l2) and torch.equal(right, r2)
    wl, _ = orf.ln_gdp(x, sc, of, wp.T, bp, wg.T, bg, mask, 1e-5)
    raw, e, r = record_error("glue ln_gdp", "left", host(left)[0], wl)
    assert e <= OUT_ATOL
    # ln_projection: w [slots, a, n], wb [a, heads]; p comes back [M, slots, n]
    w, wb = f16(rng, 4, a, 128, s=.1), f16(rng, a, 4, s=.1)
    tw, twb = dev(w, wb)
    p, hb = torch_ops.ln_projection(tx, tsc, tof, tw, twb)
    p2, hb2 = hip.ln_projection(tx, tsc, tof, layouts.slot_major(tw), layouts.heads_T(twb))
    assert p.shape == (m, 4, 128) and torch.equal(p.reshape(m, 512), p2) and torch.equal(hb, hb2)
    wp_, wb_ = orf.ln_projection(x, sc, of, w.transpose(0, 2, 1).reshape(512, a), wb.T, None, 1e-5)
    assert abs(host(p)[0].reshape(m, 512) - wp_).max() < 4e-3
    # output_projection: w [k, c]; the residual is overwritten
    o, wo, bo, res = f16(rng, m, a), f16(rng, a, ci, s=.1), f16(rng, ci, s=.1), f16(rng, m, ci)
    to, two, tbo, tres = dev(o, wo, bo, res)
    out = torch_ops.output_projection(to, two, tbo, residual=tres)
    assert out.data_ptr() == tres.data_ptr()
    want = orf.output_projection(o, wo.T, bo, res, None)
    raw, e, r = record_error("glue outproj", "out", host(out)[0], want)
    assert e <= OUT_ATOL
    # transition with AF2's leading batch axis: x [1, M, c], w1 [c, 4c], w2 [4c, c]
    c = 128
    xb = f16(rng, 1, m, c, s=2.0)
    w1, b1, w2, b2 = f16(rng, c, 4 * c, s=c ** -.5), f16(rng, 4 * c, s=.1), f16(rng, 4 * c, c, s=(4 * c) ** -.5), f16(rng, c, s=.1)
    txb, tw1, tb1, tw2, tb2 = dev(xb, w1, b1, w2, b2)
    out = torch_ops.transition(txb, tsc, tof, tw1, tb1, tw2, tb2)
    assert out.shape == (1, m, c)
    want = orf.transition(xb[0], sc, of, w1.T, b1, orf.w2_blocked(w2), b2, None, 1e-5, False)
    raw, e, r = record_error("glue transition", "out", host(out)[0][0], want)
    assert e <= OUT_ATOL
    # trimul_epilogue_ln: x_cm [ci, M] fp32, wo [ci, a], wg [a, a], written over x with add_input
    x_cm = (rng.standard_normal((ci, m)) * 20).astype(np.float32)
    lsc, lof = f32(rng, ci, mean=1.0), f32(rng, ci)
    weo, beo, wge, bge = f16(rng, ci, a, s=.1), f16(rng, a, s=.1), f16(rng, a, a, s=.1), f16(rng, a, s=.1)
    targs = dev(x_cm, lsc, lof, weo, beo, wge, bge)
    tx2 = dev(x)[0]
    out = torch_ops.trimul_epilogue_ln(targs[0], tx2, tsc, tof, targs[1], targs[2], *targs[3:], add_input=True)
    assert out.data_ptr() == tx2.data_ptr()
    want = orf.trimul_epilogue(x_cm, x, sc, of, lsc, lof, weo.T, beo, wge.T, bge, None, 1e-5, True)
    raw, e, r = record_error("glue epilogue", "out", host(out)[0], want)
    assert e <= OUT_ATOL


def test_fused_bf16_model(hip):
    """A bf16 model: bf16 activations and bf16 weights. The glue casts weights and biases to fp16
    (exact for weights of fp16 range) and keeps the activations bf16; the results are bf16 and
    agree bit for bit with the C ABI called on the fp16-cast, re-laid-out weights."""
    rng = np.random.default_rng(27)
    m, c = 4101, 128
    bf = lambda *shape, s=1.0: torch.from_numpy(rng.standard_normal(shape) * s).to(torch.bfloat16).cuda()
    x = bf(1, m, c, s=2.0)
    sc, of = (t.cuda() for t in (torch.from_numpy(f32(rng, c, mean=1.0)), torch.from_numpy(f32(rng, c))))
    w1, b1, w2, b2 = bf(c, 4 * c, s=c ** -.5), bf(4 * c, s=.1), bf(4 * c, c, s=(4 * c) ** -.5), bf(c, s=.1)
    assert torch_ops.fused_available("transition", x.dtype, c, 4 * c)
    out = torch_ops.transition(x, sc, of, w1, b1, w2, b2)
    assert out.dtype == torch.bfloat16 and out.shape == (1, m, c)
    h = lambda t: t.to(torch.float16)
    out2 = hip.transition(x.reshape(m, c), sc, of, layouts.linear_T(h(w1)), h(b1),
                          layouts.w2_blocked(h(w2)), h(b2))
    assert torch.equal(out.reshape(m, c), out2)
    w1n, w2n = h(w1).cpu().numpy(), h(w2).cpu().numpy()
    want = orf.transition(x[0].double().cpu().numpy(), sc.cpu().numpy(), of.cpu().numpy(), w1n.T,
                          h(b1).cpu().numpy(), orf.w2_blocked(w2n), h(b2).cpu().numpy(), None, 1e-5,
                          False)
    got = out[0].double().cpu().numpy()
    assert abs_excess(got, want, bf16_out=True) <= 2e-3
    # output_projection written over a bf16 residual
    o, wo, bo, res = bf(m, c), bf(c, c, s=.1), bf(c, s=.1), bf(m, c)
    res0 = res.clone()
    out = torch_ops.output_projection(o, wo, bo, residual=res)
    assert out.data_ptr() == res.data_ptr() and out.dtype == torch.bfloat16
    want = orf.output_projection(o.double().cpu().numpy(), h(wo).cpu().numpy().T,
                                 h(bo).cpu().numpy(), res0.double().cpu().numpy(), None)
    assert abs_excess(out.double().cpu().numpy(), want, bf16_out=True) <= 2e-3
