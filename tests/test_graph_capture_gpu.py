"""The command-buffer-compatible targets under HIP graph capture (the reference marks every target
but VoltaMmaBwd kCmdBufferCompatible and keeps their launch paths free of host work,
cuda/volta_mma_attn.cu:477-478). Each call is captured into one torch.cuda.CUDAGraph with its
results preallocated, the graph is replayed several times with eager calls and host syncs
between the replays, and every replay must reproduce the eager results bit for bit. The backward
that allocates nothing (clk_attention_bwd_noalloc) is captured too: capture is what it is for."""
import numpy as np
import pytest
import torch

from colabfold_legacy_kernels import layouts
from test_attention_gpu import dev, inputs

pytestmark = pytest.mark.gpu


def f16(rng, *shape, s=0.5):
    return torch.from_numpy((rng.standard_normal(shape) * s).astype(np.float16)).cuda()


def f32(rng, *shape, s=0.1, mean=0.0):
    return torch.from_numpy((rng.standard_normal(shape) * s + mean).astype(np.float32)).cuda()


def calls(hip):
    """(name, fn) pairs; fn writes into preallocated results and returns them."""
    rng = np.random.default_rng(31)
    out = []
    # attention forward, packed, packed trim
    q, k, v, bias, km, dout = dev(*inputs(4, 4, 160, 160, 32, 31))
    o, lse = torch.empty_like(q), torch.empty((4, 4, 160), dtype=torch.float32, device="cuda")
    out.append(("VoltaMma", lambda: hip.attention_fwd(q, k, v, bias, km, 32 ** -0.5, 64, 32, True,
                                                      out=o, lse=lse)))
    p = f16(rng, 6, 130, 4, 4, 32)
    pb, pkm = f16(rng, 4, 130, 130), (torch.rand(6, 130, device="cuda") > 0.2).to(torch.uint8)
    gb = f16(rng, 4 * 32, s=0.1)
    po, pto = (torch.empty((6, 130, 4, 32), dtype=torch.float16, device="cuda") for _ in range(2))
    lims = torch.tensor([130, 90, 0, 64, 130, 17, 130], dtype=torch.int32, device="cuda")
    out.append(("VoltaMmaPacked", lambda: hip.attention_packed(p, pb, pkm, gb, 32 ** -0.5, out=po)))
    out.append(("VoltaMmaPackedTrim", lambda: hip.attention_packed(p, pb, pkm, gb, 32 ** -0.5,
                                                                   lims=lims, out=pto)))
    # the no-allocation backward, on the forward's results of an eager call
    hip.attention_fwd(q, k, v, bias, km, 32 ** -0.5, 64, 32, True, out=o, lse=lse)
    o_fix, lse_fix = o.clone(), lse.clone()
    grads = (torch.empty_like(q), torch.empty_like(k), torch.empty_like(v),
             torch.empty((4, 160, 160), dtype=torch.float32, device="cuda"))
    out.append(("clk_attention_bwd_noalloc", lambda: hip.attention_bwd_noalloc(
        q, k, v, bias, km, o_fix, dout, lse_fix, 32 ** -0.5, True, grads=grads)))
    # fused ops, c = 128 and 64, with keep masks
    m, c = 5000, 128
    x, sc, of = f16(rng, m, c, s=2.0), f32(rng, c, mean=1.0), f32(rng, c)
    keep = (torch.rand(m, device="cuda") > 0.3).to(torch.float16)
    wpT, wgT, bp, bg = f16(rng, 2 * c, c, s=.1), f16(rng, 2 * c, c, s=.1), f16(rng, 2 * c, s=.1), f16(rng, 2 * c, s=.1)
    out.append(("VoltaLnGdp", lambda: hip.ln_gdp(x, sc, of, wpT, bp, wgT, bg, keep)))
    x_cm = f32(rng, c, m, s=20.0)
    woT, bo, wg2, bg2 = f16(rng, c, c, s=.1), f16(rng, c, s=.1), f16(rng, c, c, s=.1), f16(rng, c, s=.1)
    eo = torch.empty((m, c), dtype=torch.float16, device="cuda")
    out.append(("VoltaTrimulEpilogue", lambda: hip.trimul_epilogue(x_cm, x, sc, of, sc, of, woT, bo, wg2,
                                                                   bg2, keep=keep, out=eo)))
    wT, wbT = f16(rng, 512, c, s=.1), f16(rng, 4, c, s=.1)
    out.append(("VoltaLnProj", lambda: hip.ln_projection(x, sc, of, wT, wbT, keep=keep)))
    ow, ob = f16(rng, 64, c, s=.1), f16(rng, 64, s=.1)
    oo = torch.empty((m, 64), dtype=torch.float16, device="cuda")
    out.append(("VoltaOutProj", lambda: hip.output_projection(x, ow, ob, out=oo)))
    w1T, b1 = f16(rng, 4 * c, c, s=c ** -.5), f16(rng, 4 * c, s=.1)
    w2T, b2 = layouts.w2_blocked(f16(rng, 4 * c, c, s=(4 * c) ** -.5)), f16(rng, c, s=.1)
    to = torch.empty_like(x)
    out.append(("VoltaTransition", lambda: hip.transition(x, sc, of, w1T, b1, w2T, b2, keep=keep, out=to)))
    lo = torch.empty_like(x)
    out.append(("VoltaLayerNorm", lambda: hip.layer_norm(x, sc, of, out=lo)))
    gwp, gwg = f16(rng, c, 256, s=.1), f16(rng, c, 256, s=.1)
    go = torch.empty((m, 256), dtype=torch.float16, device="cuda")
    out.append(("VoltaGdp", lambda: hip.gated_dual_proj(x, gwp, bp, gwg, bg, keep, 0, out=go)))
    lhs, t, ub = f16(rng, 64, 512), f16(rng, 512, 48, 32, s=512 ** -.5), f32(rng, 32)
    norm = torch.full((64, 48), 16.0, device="cuda")
    uo = torch.empty((64, 48, 32), dtype=torch.float16, device="cuda")
    out.append(("VoltaOpmUpdate", lambda: hip.opm_update(lhs, t, ub, norm, out=uo)))
    left, right, owT = f16(rng, 16, 40, 32), f16(rng, 16, 24, 32), f16(rng, 64, 32 * 32, s=1 / 32)
    oo2 = torch.empty((40, 24, 64), dtype=torch.float16, device="cuda")
    out.append(("VoltaOpmOuter", lambda: hip.opm_outer(left, right, owT, out=oo2)))
    return out


def as_list(r):
    return [t for t in (r if isinstance(r, (tuple, list)) else (r,)) if t is not None]


def test_graph_replays_match_eager(hip):
    cases = calls(hip)
    eager = {}
    for name, fn in cases:
        eager[name] = [t.clone() for t in as_list(fn())]
    torch.cuda.synchronize()
    # capture every call into one graph, on torch's capture stream
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for name, fn in cases:  # warm up on the side stream, as torch recommends
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    results = {}
    with torch.cuda.graph(graph):
        for name, fn in cases:
            results[name] = as_list(fn())
    for replay in range(4):
        for tlist in results.values():
            for t in tlist:
                t.fill_(float("nan") if t.dtype.is_floating_point else 0)
        # eager work between replays
        cases[replay % len(cases)][1]()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, _ in cases:
            for i, (got, want) in enumerate(zip(results[name], eager[name])):
                assert torch.equal(got, want), "%s result %d differs on replay %d" % (name, i, replay)
