"""Write guards: every result of the attention and fused entry points is written into the middle of
a larger buffer filled with a sentinel bit pattern, and the call must leave every sentinel in
place, so a store past either end of a result (which an exactly sized torch tensor would hide in
the caching allocator's slack) fails the test without faulting. The guarded call's results must
also be bit-identical to those of the same call on exactly sized tensors.

The reference runs each packed case in a process of its own with one allocation per array
(tests/test_packed_attention.py:5-7, 105-106); the guards here check the same property, stores
inside each result's bounds, on the ragged shapes where a tile overhangs the end: attention at
70 x 83 (D = 16), Sq = Sk = 130 (D = 32, 64) and 1000 x 700 (D = 96, the query-window backward),
the packed forward on a 70-residue pair, and the fused ops at 59 and 4101 rows, fp16 and bf16.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

PAD = 4096  # guard elements on each side (16-byte aligned for every result type)
_BITS = {torch.float16: (torch.int16, 0x5A5A), torch.bfloat16: (torch.int16, 0x5A5A),
         torch.float32: (torch.int32, 0x5A5A5A5A)}


class Guarded:
    """A result tensor of `shape` inside a sentinel-filled buffer."""

    def __init__(self, shape, dtype):
        self.n = int(np.prod(shape))
        self.buf = torch.empty(PAD + self.n + PAD, dtype=dtype, device="cuda")
        itype, pattern = _BITS[dtype]
        self.bits = self.buf.view(itype)
        self.pattern = pattern
        self.bits.fill_(pattern)
        self.t = self.buf[PAD:PAD + self.n].view(shape)

    def intact(self):
        torch.cuda.synchronize()
        before = bool((self.bits[:PAD] == self.pattern).all())
        after = bool((self.bits[PAD + self.n:] == self.pattern).all())
        return before and after


def same_bits(a, b):
    torch.cuda.synchronize()
    if a.dtype == torch.float32:
        return bool(torch.equal(a.view(torch.int32), b.view(torch.int32)))
    return bool(torch.equal(a.view(torch.int16), b.view(torch.int16)))


def assert_guarded(pairs, label):
    for name, g, plain in pairs:
        assert g.intact(), "%s: a store landed outside %s" % (label, name)
        assert same_bits(g.t, plain), "%s: %s differs from the call on exact tensors" % (label, name)


def gen(shape, seed, s=0.5, dtype=torch.float16):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return (torch.randn(shape, generator=g, device="cuda") * s).to(dtype)


ATTN_SHAPES = [dict(n=3, h=4, sq=70, sk=83, d=16), dict(n=2, h=2, sq=130, sk=130, d=32),
               dict(n=2, h=2, sq=130, sk=130, d=64), dict(n=2, h=1, sq=1000, sk=700, d=96)]


@pytest.mark.parametrize("kw", ATTN_SHAPES, ids=lambda kw: "%dx%d_d%d" % (kw["sq"], kw["sk"], kw["d"]))
def test_attention_results_stay_in_bounds(hip, kw):
    n, h, sq, sk, d = kw["n"], kw["h"], kw["sq"], kw["sk"], kw["d"]
    print("guards attention", kw, flush=True)
    q, k, v = gen((n, h, sq, d), 1), gen((n, h, sk, d), 2), gen((n, h, sk, d), 3)
    bias, dout = gen((h, sq, sk), 4), gen((n, h, sq, d), 5)
    g = torch.Generator(device="cuda")
    g.manual_seed(6)
    km = (torch.rand((n, sk), generator=g, device="cuda") > 0.15).to(torch.uint8)
    scale = d ** -0.5
    bq, bk = (64, 64) if d == 64 else (64, 32)  # entries of the forward's (D, bq, bk) table
    out, lse = hip.attention_fwd(q, k, v, bias, km, scale, bq, bk)
    grads = hip.attention_bwd(q, k, v, bias, km, out, dout, lse, scale, want_dbias=True)
    gout, glse = Guarded(out.shape, torch.float16), Guarded(lse.shape, torch.float32)
    hip.attention_fwd(q, k, v, bias, km, scale, bq, bk, out=gout.t, lse=glse.t)
    gg = [Guarded(t.shape, t.dtype) for t in grads]
    hip.attention_bwd(q, k, v, bias, km, out, dout, lse, scale, want_dbias=True,
                      grads=tuple(x.t for x in gg))
    assert_guarded([("out", gout, out), ("lse", glse, lse)] +
                   [(name, x, t) for name, x, t in zip(("dq", "dk", "dv", "dbias"), gg, grads)],
                   str(kw))


@pytest.mark.parametrize("column", (False, True))
@pytest.mark.parametrize("gated", (False, True))
def test_packed_results_stay_in_bounds(hip, column, gated):
    s, h, d = 70, 4, 32
    slots = 4 if gated else 3
    p = gen((s, s, slots, h, d), 7)
    bias = gen((h, s, s), 8)
    km = torch.ones((s, s), dtype=torch.uint8, device="cuda")
    km[:, -5:] = 0
    gate_bias = gen((h, d), 9)
    out = hip.attention_packed(p, bias, km, gate_bias, d ** -0.5, column=column)
    gout = Guarded(out.shape, torch.float16)
    hip.attention_packed(p, bias, km, gate_bias, d ** -0.5, column=column, out=gout.t)
    assert_guarded([("out", gout, out)], "packed column=%s gated=%s" % (column, gated))


FUSED_ROWS = (59, 4101)
ACTS = (torch.float16, torch.bfloat16)


def _lib_call(hip, name, tensors, *attrs):
    bufs = [hip.buffer(t) for t in tensors]
    hip._check(getattr(hip.lib(), name)(hip._stream(tensors[0]), *map(hip._ref, bufs), *attrs))


@pytest.mark.parametrize("dt", ACTS, ids=("f16", "bf16"))
@pytest.mark.parametrize("c", (64, 128))
@pytest.mark.parametrize("m", FUSED_ROWS)
def test_fused_results_stay_in_bounds(hip, m, c, dt):
    print("guards fused m=%d c=%d %s" % (m, c, dt), flush=True)
    f = lambda shape, seed, s=0.5: gen(shape, seed, s)  # fp16 weights and biases
    f32 = lambda shape, seed, mean=0.0: gen(shape, seed, 0.1, torch.float32) + mean
    x = gen((m, c), 11, 2.0, dt)
    sc, of = f32((c,), 12, 1.0), f32((c,), 13)
    label = "m=%d c=%d %s" % (m, c, dt)

    # ln_gdp: left, right [c, m]
    wpT, wgT, bp, bg = f((2 * c, c), 14, .1), f((2 * c, c), 15, .1), f((2 * c,), 16, .1), f((2 * c,), 17, .1)
    mask = (gen((m,), 18, 1.0, torch.float32) > -1.0).to(torch.float16)
    left, right = hip.ln_gdp(x, sc, of, wpT, bp, wgT, bg, mask)
    gl, gr = Guarded(left.shape, dt), Guarded(right.shape, dt)
    _lib_call(hip, "clk_ln_gdp", [x, sc, of, wpT, bp, wgT, bg, mask, gl.t, gr.t], 1e-5)
    assert_guarded([("left", gl, left), ("right", gr, right)], label + " ln_gdp")

    # ln_projection: p [m, 512], bias [4, m]
    wT, wbT = f((512, c), 19, .1), f((4, c), 20, .1)
    p, b = hip.ln_projection(x, sc, of, wT, wbT)
    gp, gb = Guarded(p.shape, dt), Guarded(b.shape, dt)
    one = torch.zeros(1, dtype=torch.float16, device="cuda")
    _lib_call(hip, "clk_ln_projection", [x, sc, of, wT, wbT, one, gp.t, gb.t], 1e-5, 512, 4, 0)
    assert_guarded([("p", gp, p), ("bias", gb, b)], label + " ln_projection")

    # trimul_epilogue: out [m, c]
    x_cm = gen((c, m), 21, 1.0, torch.float32)
    lns, lno = f32((c,), 22, 1.0), f32((c,), 23)
    woT, bo, wgT2, bg2 = f((c, c), 24, .1), f((c,), 25, .1), f((c, c), 26, .1), f((c,), 27, .1)
    e = hip.trimul_epilogue(x_cm, x, sc, of, lns, lno, woT, bo, wgT2, bg2)
    ge = Guarded(e.shape, dt)
    hip.trimul_epilogue(x_cm, x, sc, of, lns, lno, woT, bo, wgT2, bg2, out=ge.t)
    assert_guarded([("out", ge, e)], label + " trimul_epilogue")

    # output_projection: out [m, c] from o [m, 128], with a residual
    o, r = gen((m, 128), 28, 1.0, dt), gen((m, c), 29, 1.0, dt)
    wo, b3 = f((c, 128), 30, .1), f((c,), 31, .1)
    y = hip.output_projection(o, wo, b3, residual=r)
    gy = Guarded(y.shape, dt)
    hip.output_projection(o, wo, b3, residual=r, out=gy.t)
    assert_guarded([("out", gy, y)], label + " output_projection")

    # transition: out [m, c], hidden 4c
    w1T, b1 = f((4 * c, c), 32, c ** -.5), f((4 * c,), 33, .1)
    w2T, b2 = f((4 * c // 64, c, 64), 34, (4 * c) ** -.5), f((c,), 35, .1)
    t = hip.transition(x, sc, of, w1T, b1, w2T, b2)
    gt = Guarded(t.shape, dt)
    hip.transition(x, sc, of, w1T, b1, w2T, b2, out=gt.t)
    assert_guarded([("out", gt, t)], label + " transition")
