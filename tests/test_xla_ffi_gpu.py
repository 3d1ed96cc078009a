"""The XLA FFI handler symbols on the GPU, called with real buffers through a mock of the XLA API
(stream from XLA_FFI_Stream_Get, backward scratch from XLA_FFI_DeviceMemory_Allocate): every
handler's results are bit-identical to the C entry point it wraps, called through
colabfold_legacy_kernels.hip on the same inputs."""
import ctypes

import numpy as np
import pytest
import torch

import ffi_frames as ff

pytestmark = pytest.mark.gpu

CODE = {torch.float16: ff.F16, torch.float32: ff.F32, torch.uint8: ff.U8, torch.int32: ff.S32}


def b(t):
    return (CODE[t.dtype], t.data_ptr(), tuple(t.shape))


def mock():
    held = []

    def allocate(size, align):
        t = torch.empty(size + align, dtype=torch.uint8, device="cuda")
        held.append(t)
        return (t.data_ptr() + align - 1) // align * align

    m = ff.MockXla(stream=torch.cuda.current_stream().cuda_stream, allocate=allocate)
    m.held = held
    return m


def same(a, c):
    torch.cuda.synchronize()
    return np.array_equal(a.cpu().numpy(), c.cpu().numpy())


def g(*shape, s=1.0, dtype=torch.float16, mean=0.0):
    return (torch.randn(shape, device="cuda") * s + mean).to(dtype)


def test_attention_handlers(hip):
    torch.manual_seed(0)
    lib = hip.lib()
    n, h, s, d = 2, 2, 96, 32
    q, k, v, dout = g(n, h, s, d, s=.5), g(n, h, s, d, s=.5), g(n, h, s, d), g(n, h, s, d)
    bias = g(h, s, s, s=.5)
    kmask = (torch.rand(n, s, device="cuda") > .2).to(torch.uint8)
    scale = d ** -0.5
    out_ref, lse_ref = hip.attention_fwd(q, k, v, bias, kmask, scale, 64, 32, True)
    out, lse = torch.empty_like(q), torch.empty((n, h, s), device="cuda")
    m = mock()
    attrs = {"scale": (ff.F32, scale), "block_q": (ff.S64, 64), "block_k": (ff.S64, 32),
             "want_lse": (ff.PRED, 1)}
    assert m.call(lib.VoltaMma, [b(q), b(k), b(v), b(bias), b(kmask)], [b(out), b(lse)], attrs) is None
    assert not m.errors and same(out, out_ref) and same(lse, lse_ref)

    ref = hip.attention_bwd(q, k, v, bias, kmask, out_ref, dout, lse_ref, scale, True)
    grads = [torch.empty_like(q), torch.empty_like(k), torch.empty_like(v),
             torch.empty((h, s, s), device="cuda")]
    attrs = {"scale": (ff.F32, scale), "want_dbias": (ff.PRED, 1)}
    args = [b(t) for t in (q, k, v, bias, kmask, out_ref, dout, lse_ref)]
    assert m.call(lib.VoltaMmaBwd, args, [b(t) for t in grads], attrs) is None
    assert not m.errors and len(m.allocations) == 1 and len(m.frees) == 1
    for name, x, y in zip(("dq", "dk", "dv", "dbias"), grads, ref):
        assert same(x, y), name


@pytest.mark.parametrize("column", [False, True])
def test_packed_handlers(hip, column):
    torch.manual_seed(1)
    lib = hip.lib()
    X, Y, H, D = 3, 40, 2, 32
    p = g(X, Y, 4, H, D, s=.5)
    S = X if column else Y
    N = Y if column else X
    bias = g(H, S, S, s=.5)
    kmask = (torch.rand(N, S, device="cuda") > .2).to(torch.uint8)
    gate_bias = g(H * D, s=.1)
    scale = D ** -0.5
    ref = hip.attention_packed(p, bias, kmask, gate_bias, scale, column=column)
    lims_np = np.zeros(N + 1, np.int32)
    km = kmask.cpu().numpy()
    for i in range(N):
        live = np.nonzero(km[i])[0]
        lims_np[i] = live[-1] + 1 if len(live) else 0
    lims_np[N] = lims_np[:N].max()
    lims = torch.from_numpy(lims_np).cuda()
    ref_trim = hip.attention_packed(p, bias, kmask, gate_bias, scale, column=column, lims=lims)
    m = mock()
    attrs = {"scale": (ff.F32, scale), "block_q": (ff.S64, 64), "block_k": (ff.S64, 32),
             "column": (ff.PRED, int(column))}
    out = torch.empty_like(ref)
    assert m.call(lib.VoltaMmaPacked, [b(p), b(bias), b(kmask), b(gate_bias)], [b(out)], attrs) is None
    assert not m.errors and same(out, ref)
    out = torch.empty_like(ref)
    assert m.call(lib.VoltaMmaPackedTrim, [b(p), b(bias), b(kmask), b(gate_bias), b(lims)], [b(out)],
                  attrs) is None
    assert not m.errors and same(out, ref_trim)


def test_fused_handlers(hip):
    torch.manual_seed(2)
    lib = hip.lib()
    M, c = 200, 64
    x, sc, of = g(M, c, s=2.), g(c, s=.1, mean=1., dtype=torch.float32), g(c, s=.1, dtype=torch.float32)
    keep = torch.ones(M, dtype=torch.float16, device="cuda")
    keep[64:128] = 0
    m = mock()

    wpT, bp, wgT, bg = g(2 * c, c, s=.1), g(2 * c, s=.1), g(2 * c, c, s=.1), g(2 * c, s=.1)
    left_ref, right_ref = hip.ln_gdp(x, sc, of, wpT, bp, wgT, bg, keep)
    left, right = torch.empty_like(left_ref), torch.empty_like(right_ref)
    assert m.call(lib.VoltaLnGdp, [b(t) for t in (x, sc, of, wpT, bp, wgT, bg, keep)], [b(left), b(right)],
                  {"eps": (ff.F32, 1e-5)}) is None
    assert same(left, left_ref) and same(right, right_ref)

    x_cm = g(c, M, s=3., dtype=torch.float32)
    woT, bo, wgT2, bg2 = g(c, c, s=.1), g(c, s=.1), g(c, c, s=.1), g(c, s=.1)
    ref = hip.trimul_epilogue(x_cm, x, sc, of, sc, of, woT, bo, wgT2, bg2, keep=keep)
    out = torch.empty_like(ref)
    attrs = {"eps": (ff.F32, 1e-5), "add_input": (ff.PRED, 0), "has_keep": (ff.PRED, 1)}
    assert m.call(lib.VoltaTrimulEpilogue, [b(t) for t in (x_cm, x, sc, of, sc, of, woT, bo, wgT2, bg2, keep)],
                  [b(out)], attrs) is None
    assert same(out, ref)

    wT, wbT = g(128, c, s=.1), g(4, c, s=.1)
    p_ref, hb_ref = hip.ln_projection(x, sc, of, wT, wbT, keep=keep)
    p, hb = torch.empty_like(p_ref), torch.empty_like(hb_ref)
    attrs = {"eps": (ff.F32, 1e-5), "n": (ff.S64, 128), "heads": (ff.S64, 4), "has_keep": (ff.PRED, 1)}
    assert m.call(lib.VoltaLnProj, [b(t) for t in (x, sc, of, wT, wbT, keep)], [b(p), b(hb)], attrs) is None
    assert same(p, p_ref) and same(hb, hb_ref)

    # with a residual the output stands in for it: padding rows keep what it held
    o, w, bb, res = g(M, 128), g(c, 128, s=.1), g(c, s=.1), g(M, c)
    ref = hip.output_projection(o, w, bb, residual=res, keep=keep, out=res.clone())
    out = res.clone()
    attrs = {"has_residual": (ff.PRED, 1), "has_keep": (ff.PRED, 1)}
    assert m.call(lib.VoltaOutProj, [b(t) for t in (o, w, bb, res, keep)], [b(out)], attrs) is None
    assert same(out, ref)

    w1T, b1, w2T, b2 = g(4 * c, c, s=.1), g(4 * c, s=.1), g(4, c, 64, s=.05), g(c, s=.1)
    ref = hip.transition(x, sc, of, w1T, b1, w2T, b2, keep=keep)
    out = torch.empty_like(ref)
    attrs = {"eps": (ff.F32, 1e-5), "add_input": (ff.PRED, 0), "has_keep": (ff.PRED, 1)}
    assert m.call(lib.VoltaTransition, [b(t) for t in (x, sc, of, w1T, b1, w2T, b2, keep)], [b(out)],
                  attrs) is None
    assert same(out, ref)
    assert not m.errors


def test_plain_handlers(hip):
    torch.manual_seed(3)
    lib = hip.lib()
    M, K, N = 150, 64, 96
    x = g(M, K)
    sc, of = g(K, s=.1, mean=1., dtype=torch.float32), g(K, s=.1, dtype=torch.float32)
    m = mock()
    ref = hip.layer_norm(x, sc, of, 1e-5)
    out = torch.empty_like(ref)
    assert m.call(lib.VoltaLayerNorm, [b(x), b(sc), b(of)], [b(out)], {"eps": (ff.F32, 1e-5)}) is None
    assert same(out, ref)
    wp, wg, bp, bg = g(K, N, s=.1), g(K, N, s=.1), g(N, s=.1), g(N, s=.1)
    mask = torch.ones(M, dtype=torch.float16, device="cuda")
    for act in (0, 1):
        ref = hip.gated_dual_proj(x, wp, bp, wg, bg, mask, activation=act)
        out = torch.empty_like(ref)
        assert m.call(lib.VoltaGdp, [b(t) for t in (x, wp, bp, wg, bg, mask)], [b(out)],
                      {"activation": (ff.S64, act)}) is None
        assert same(out, ref)
    assert not m.errors


def test_opm_handlers(hip):
    torch.manual_seed(4)
    lib = hip.lib()
    B, K, D, F, C = 37, 64, 64, 128, 32
    lhs, t = g(B, K), g(K, D, F, s=K ** -.5)
    bias = g(F, s=.1, dtype=torch.float32)
    norm = torch.randint(1, 3, (B, D), device="cuda").float()
    res = g(B, D, F)
    m = mock()
    for residual in (None, res):
        ref = hip.opm_update(lhs, t, bias, norm, residual, eps=1e-3)
        out = torch.empty_like(ref)
        rarg = residual if residual is not None else torch.zeros(1, dtype=torch.float16, device="cuda")
        assert m.call(lib.VoltaOpmUpdate, [b(x) for x in (lhs, t, bias, norm, rarg)], [b(out)],
                      {"eps": (ff.F32, 1e-3), "has_residual": (ff.PRED, int(residual is not None))}) is None
        assert same(out, ref)
    left, right, wT = g(16, B, C), g(16, D, 32), g(F, 32 * C, s=1 / 32)
    ref = hip.opm_outer(left, right, wT)
    out = torch.empty_like(ref)
    assert m.call(lib.VoltaOpmOuter, [b(left), b(right), b(wT)], [b(out)], {}) is None
    assert same(out, ref)
    assert not m.errors
