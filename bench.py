#!/usr/bin/env python3
"""Benchmark of the ColabFold legacy-kernel hot path on one MI355X (gfx950).

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-fused] [--no-packed]
                  [--no-extra] [--calibration-copy MIB]
  python bench.py --stats-summary DIR            (text summary of a rocprofv3 --stats run)
  python bench.py --traffic-summary FETCH_DIR WRITE_DIR [--calibration-copy MIB] [--prefix c2:]
                                                 (HBM bytes per dispatch from two --pmc runs)
  python bench.py --only c2|c5 ...                (profiling: that config's object alone)
  python bench.py --counter-summary DIR [DIR ...] (per-kernel means of the counters of --pmc runs)

A step is one attention forward + backward of BASELINE config C3 (MSA row attention with pair
bias, fp16: N_seq = 512 rows, N_res = 384, H = 8, D = 32): VoltaMma(want_lse) then
VoltaMmaBwd(want_dbias), through the library's C ABI on the current stream, inputs already in
HBM. value is the step's algorithmic TFLOP/s (14 u flops, u = N H S^2 D: forward 4u, backward
10u with its recompute of S). The other GPU configs of BASELINE.json are reported beside it as
objects of the same line: "c2" (triangle attention fwd + bwd, N_res = 256) and "c5" (triangle
attention forward, N_res = 1024, want_lse off), each with its kernels and roofline. ms_per_step
is timed over steps launched back to back with nothing else in the stream; per-kernel durations
come from as many more steps with HIP events that the library records on its launch stream at
its kernel boundaries (clk_set_stage_events), whose own step time is ms_per_step_staged (each
event record adds a few microseconds of device time). The roofline object is the
dominant kernel's, its "traffic" the HBM bytes per dispatch that the committed rocprofv3 counter
summaries (profiles/attention_c3_traffic.txt, profiles/attention_c2_c5_traffic.txt) measured for
that kernel at that config. Reported beside the step:
the gated packed forward VoltaMmaPacked (G = 4) on the same shape, and the fused pair-stack ops
of config C4 (M = 262144 rows, c = 64 and 128), the unfused LayerNorm and gated dual projection
at c = 128 on the same rows, and the outer product mean pair on C3's residues (B = D = 384, 16 MSA
rows of 32 channels, F = 128), each timed over enough rotating buffer sets that no call finds its
inputs in the 256 MB Infinity Cache. cpu_baseline is the fp32 torch-CPU
restatement of the reference tests' jnp attention (oracle/cpu_ref.py; jax is not installed) on a
bounded row sample of the same workload, on this box's host cores.

One GPU per box here: --gpus above 1 exits with a message.
"""
import argparse
import csv
import ctypes
import glob
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "colabfold-legacy-kernels_amd"))
sys.path.insert(0, ROOT)

METRIC = "ms/call + TFLOP/s attn fwd+bwd (N_res=384); fused LN-proj GB/s, 1 GPU"
PEAK_TFLOPS = 2516.6   # MI355X dense fp16 MFMA (256 CU x 2.4 GHz x 4096 flop/clk)
PEAK_GBS = 8000.0      # MI355X HBM3E
MALL_BYTES = 256 << 20
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "attention_c3_traffic.txt")
# C2's and C5's kernels, with stage names prefixed "c2:" / "c5:"
EXTRA_TRAFFIC_FILE = os.path.join(ROOT, "profiles", "attention_c2_c5_traffic.txt")

N, H, S, D = 512, 8, 384, 32
FWD_STAGES = ("attn_fwd",)
BWD_STAGES = ("bwd_biast", "bwd_dq", "bwd_dkdv", "bwd_dbias")
# kernel-name fragment in a rocprofv3 record -> the bench's stage name
KERNEL_STAGES = (("attn_fwd_kernel", "attn_fwd"), ("attn_bwd_biast_kernel", "bwd_biast"),
                 ("attn_bwd_dq_kernel", "bwd_dq"), ("attn_bwd_dkdv_kernel", "bwd_dkdv"),
                 ("attn_bwd_dkdv_reg_kernel", "bwd_dkdv"), ("attn_bwd_dkdv_reg3_kernel", "bwd_dkdv"),
                 ("attn_bwd_dkdv_sum_kernel", "bwd_dkdv_sum"),
                 ("attn_bwd_dbias_kernel", "bwd_dbias"))
CALIBRATION_KERNEL = "bitwise_not"


class HipEvents:
    """hipEvent_t handles through libamdhip64, for the library's stage hook."""

    def __init__(self):
        self.hip = ctypes.CDLL("libamdhip64.so")
        self.hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                                 ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]

    def create(self, n):
        evs = []
        for _ in range(n):
            e = ctypes.c_void_p()
            if self.hip.hipEventCreate(ctypes.byref(e)) != 0:
                raise RuntimeError("hipEventCreate failed")
            evs.append(e)
        return evs

    def elapsed_ms(self, a, b):
        ms = ctypes.c_float()
        if self.hip.hipEventElapsedTime(ctypes.byref(ms), a, b) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value

    def destroy(self, evs):
        for e in evs:
            self.hip.hipEventDestroy(e)


def arm(hip, evs):
    arr = (ctypes.c_void_p * max(len(evs), 1))(*[e.value for e in evs])
    if hip.lib().clk_set_stage_events(arr, len(evs)) != 0:
        raise RuntimeError(hip.lib().clk_last_error().decode())


def disarm(hip):
    hip.lib().clk_set_stage_events(None, 0)


def roof_entry(ms_list, flops, byts, mean=None, **extra):
    """Per-kernel timing against both roofs; the bound is the larger ideal time. `mean` replaces
    the mean of ms_list where the caller timed the calls another way."""
    med = statistics.median(ms_list)
    mean = statistics.mean(ms_list) if mean is None else mean
    t_mfma = flops / (PEAK_TFLOPS * 1e12) * 1e3
    t_hbm = byts / (PEAK_GBS * 1e9) * 1e3
    e = {"ms": round(mean, 5), "ms_median": round(med, 5), "calls": len(ms_list),
         "tflops": round(flops / mean / 1e9, 2), "gbs": round(byts / mean / 1e6, 1),
         "bound": "mfma" if t_mfma > t_hbm else "hbm",
         "frac": round(max(t_mfma, t_hbm) / mean, 4), "frac_mfma": round(t_mfma / mean, 4),
         "frac_hbm": round(t_hbm / mean, 4), "algo_flops": flops, "algo_bytes": byts}
    e.update(extra)
    return e


def attention_algo(ws_bytes, n=N, h=H, s=S, d=D):
    """(flops, bytes, scratch bytes) per launch of each attention kernel at [n, h, s, d]. Bytes
    count every tensor of the kernel's contract read or written once; implementation scratch is
    listed apart (scratch_bytes)."""
    u = float(n) * h * s * s * d
    t = n * h * s * d * 2                   # one fp16 [N,H,S,D] tensor
    row = n * h * s * 4                     # one fp32 [N,H,S] row statistic
    bias, km, dbias = h * s * s * 2, n * s, h * s * s * 4
    sqa, ska = -(-s // 32) * 32, -(-s // 64) * 64
    # the workspace: two query-term rows, the transposed log2e bias (fp32, one masked-logit row
    # per head, queries padded to 32 QT where the register dK/dV kernel runs), the dBias partials
    # (with any window sums) and the dQ kernel's fp16 bias fragments
    r256 = lambda b: -(-b // 256) * 256
    qt = sqa // 32
    sqb = 32 * (4 if qt <= 4 else 8 if qt <= 8 else 12) if d == 32 and qt <= 12 else sqa
    biast = h * (ska + 1) * sqb * 4
    bfrag = h * sqa * ska * 2
    partial = max(ws_bytes - 2 * r256(n * h * sqa * 4) - r256(biast) - r256(bfrag), 0)
    return {
        "attn_fwd": (4 * u, 3 * t + bias + km + t + row, 0),
        "bwd_biast": (0.0, bias + biast + bfrag, 0),
        # dQ = dS K is 2u; the kernel also recomputes S and dP (4u more)
        "bwd_dq": (2 * u, 5 * t + row + bias + km + t, 2 * row + bfrag),
        "bwd_dkdv": (8 * u, 4 * t + row + bias + km + 2 * t, partial),
        "bwd_dbias": (0.0, dbias, partial),
    }


def attention_sets(torch, hip, n, h, s, d, mask_frac, bias_std, seed, backward, want_lse):
    """Two resident buffer sets for one attention config (a step never finds the previous
    step's tensors in the MALL). mask_frac > 0 pads that share of residues on both axes
    (kmask = res (x) res, the triangle-attention mask)."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    sets = []
    for _ in range(2):
        q, k, v, dout = (torch.randn((n, h, s, d), generator=g, device="cuda").half() for _ in range(4))
        bias = (torch.randn((h, s, s), generator=g, device="cuda") * bias_std).half()
        if mask_frac > 0:
            dead = torch.randperm(s, generator=torch.Generator().manual_seed(seed))[:round(mask_frac * s)]
            res = torch.ones(s, dtype=torch.uint8)
            res[dead] = 0
            kmask = (res[:, None] * res[None, :]).contiguous().cuda() if n == s else \
                res[None, :].expand(n, s).contiguous().cuda()
        else:
            kmask = torch.ones((n, s), dtype=torch.uint8, device="cuda")
        out = torch.empty_like(q)
        lse = (torch.empty((n, h, s), dtype=torch.float32, device="cuda") if want_lse
               else torch.zeros(1, dtype=torch.float32, device="cuda"))
        ws = grads = None
        if backward:
            ws = torch.empty(hip.attention_bwd_workspace(q, k), dtype=torch.uint8, device="cuda")
            grads = (torch.empty_like(q), torch.empty_like(k), torch.empty_like(v),
                     torch.empty((h, s, s), dtype=torch.float32, device="cuda"))
        else:
            del dout
            dout = None
        sets.append((q, k, v, bias, kmask, dout, out, lse, ws, grads))
    return sets


def bench_attention(torch, hip, steps, warmup, ev, n=N, h=H, s=S, d=D, mask_frac=0.0, bias_std=1.0,
                    seed=0, backward=True, want_lse=True):
    """ms per step (VoltaMma, then VoltaMmaBwd(want_dbias) when `backward`), the step's
    algorithmic flops, per-kernel timings from the library's stage events, and ms per step with
    those events armed. The step time comes from `steps` steps launched back to back between two
    events, with no stage events in the stream (each event record the library makes at a kernel
    boundary adds a few microseconds of device time); the per-kernel timings from `steps` more
    steps with them armed."""
    u = float(n) * h * s * s * d
    scale = d ** -0.5
    sets = attention_sets(torch, hip, n, h, s, d, mask_frac, bias_std, seed, backward, want_lse)

    def step(st, fwd_ev=None, bwd_ev=None):
        q, k, v, bias, kmask, dout, out, lse, ws, grads = st
        if fwd_ev:
            arm(hip, fwd_ev)
        hip.attention_fwd(q, k, v, bias, kmask, scale, 64, 32, want_lse, out=out, lse=lse)
        if backward:
            if bwd_ev:
                arm(hip, bwd_ev)
            hip.attention_bwd(q, k, v, bias, kmask, out, dout, lse, scale, True, workspace=ws,
                              grads=grads)
        if fwd_ev or bwd_ev:
            disarm(hip)

    bwd_stages = BWD_STAGES if backward else ()
    for i in range(warmup):
        step(sets[i % 2])
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for i in range(steps):
        step(sets[i % 2])
    stop.record()
    torch.cuda.synchronize()
    plain_ms = start.elapsed_time(stop)
    fwd_evs = [ev.create(len(FWD_STAGES) + 1) for _ in range(steps)]
    bwd_evs = [ev.create(len(bwd_stages) + 1) if backward else None for _ in range(steps)]
    torch.cuda.synchronize()
    start.record()
    for i in range(steps):
        step(sets[i % 2], fwd_evs[i], bwd_evs[i])
    stop.record()
    torch.cuda.synchronize()
    staged_ms = start.elapsed_time(stop)
    per = {name: [] for name in FWD_STAGES + bwd_stages}
    for fe, be in zip(fwd_evs, bwd_evs):
        for i, name in enumerate(FWD_STAGES):
            per[name].append(ev.elapsed_ms(fe[i], fe[i + 1]))
        for i, name in enumerate(bwd_stages):
            per[name].append(ev.elapsed_ms(be[i], be[i + 1]))
    for e in fwd_evs + [b for b in bwd_evs if b]:
        ev.destroy(e)
    disarm(hip)

    ws_bytes = sets[0][8].numel() if backward else 0
    algo = attention_algo(ws_bytes, n, h, s, d)
    kernels = {name: roof_entry(per[name], algo[name][0], algo[name][1], scratch_bytes=algo[name][2])
               for name in per}
    return plain_ms / steps, (14 if backward else 4) * u, kernels, staged_ms / steps


def roofline_of(kernels, prefix=""):
    """The roofline object of the dominant (longest) kernel of a step; `prefix` names the config
    whose profiled traffic applies ("" for C3, "c2:" or "c5:")."""
    dom = max(kernels, key=lambda k: kernels[k]["ms"])
    kd = kernels[dom]
    if kd["bound"] == "mfma":
        roof = {"bound": "mfma", "achieved": kd["tflops"], "peak": PEAK_TFLOPS, "unit": "TFLOP/s"}
    else:
        roof = {"bound": "hbm", "achieved": kd["gbs"], "peak": PEAK_GBS, "unit": "GB/s"}
    roof["frac"] = round(roof["achieved"] / roof["peak"], 4)
    roof["traffic"] = load_traffic(prefix + dom)
    roof["kernel"] = dom
    roof["ms"] = kd["ms"]
    return roof


# the two other GPU configs of BASELINE.json, reported beside the C3 headline:
# C2 triangle attention fwd+bwd (N_res = 256, H = 4, bias ~ N(0, 0.5), 5% of residues padded on
# both axes) and C5 triangle attention forward only (N_res = 1024, H = 4, 8% padded, no lse)
EXTRA_CONFIGS = {
    "c2": dict(n=256, h=4, s=256, d=32, mask_frac=0.05, bias_std=0.5, seed=2, backward=True,
               want_lse=True,
               workload="C2: triangle attention (starting node), fwd (want_lse) + bwd (want_dbias)"),
    "c5": dict(n=1024, h=4, s=1024, d=32, mask_frac=0.08, bias_std=1.0, seed=5, backward=False,
               want_lse=False, workload="C5: triangle attention forward, N_res = 1024, want_lse off"),
}


def bench_extra(torch, hip, ev, name, steps, warmup):
    cfg = dict(EXTRA_CONFIGS[name])
    workload = cfg.pop("workload")
    ms, flops, kernels, staged = bench_attention(torch, hip, steps, warmup, ev, **cfg)
    t_mfma = flops / (PEAK_TFLOPS * 1e12) * 1e3
    torch.cuda.empty_cache()
    return {"workload": workload, "shape": [cfg["n"], cfg["h"], cfg["s"], cfg["d"]],
            "ms_per_step": round(ms, 5), "ms_per_step_staged": round(staged, 5),
            "tflops": round(flops / ms / 1e9, 2),
            "frac_mfma_step": round(t_mfma / ms, 4), "flops_per_step": flops,
            "roofline": roofline_of(kernels, name + ":"), "kernels": kernels}


def bench_packed(torch, hip, iters, warmup, ev):
    """VoltaMmaPacked (G = 4: q, k, v and the gate in one [X, Y, 4, H, D] tensor) on C3's shape."""
    u = float(N) * H * S * S * D
    g = torch.Generator(device="cuda")
    g.manual_seed(2)
    sets = []
    for _ in range(2):
        p = torch.randn((N, S, 4, H, D), generator=g, device="cuda").half()
        bias = torch.randn((H, S, S), generator=g, device="cuda").half()
        kmask = torch.ones((N, S), dtype=torch.uint8, device="cuda")
        gate_bias = torch.zeros(H * D, dtype=torch.float16, device="cuda")
        out = torch.empty((N, S, H, D), dtype=torch.float16, device="cuda")
        sets.append((p, bias, kmask, gate_bias, out))
    calls = [lambda st=st: hip.attention_packed(st[0], st[1], st[2], st[3], D ** -0.5, out=st[4])
             for st in sets]
    plain = time_calls(torch, calls, iters, warmup)
    evs = [ev.create(2) for _ in range(iters)]
    for i in range(iters):
        p, bias, kmask, gb, out = sets[i % 2]
        arm(hip, evs[i])
        hip.attention_packed(p, bias, kmask, gb, D ** -0.5, out=out)
    disarm(hip)
    torch.cuda.synchronize()
    ms = [ev.elapsed_ms(e[0], e[1]) for e in evs]
    for e in evs:
        ev.destroy(e)
    t = N * H * S * D * 2
    # ms: calls back to back with no events between them; ms_median and ms_staged: per call,
    # with the library's stage events armed
    return roof_entry(ms, 4 * u, 4 * t + H * S * S * 2 + N * S + t + H * D * 2,
                      mean=statistics.mean(plain), ms_staged=round(statistics.mean(ms), 5))


def fused_bytes_flops(op, m, c, n=None, heads=0):
    """Algorithmic HBM bytes (activations read and results written once, weights excluded) and
    flops per call of a fused op at width c over m rows."""
    if op == "ln_gdp":
        p = 2 * c
        return float(m * c * 2 + m * 2 + m * p * 2), 2.0 * m * c * (2 * p)
    if op == "trimul_epilogue":
        return float(m * c * 4 + m * c * 2 + m * c * 2), 2.0 * m * c * c * 2
    if op == "ln_projection":
        return float(m * c * 2 + m * n * 2 + m * heads * 2), 2.0 * m * c * (n + heads)
    if op == "output_projection":
        return float(m * n * 2 + m * c * 2 * 2), 2.0 * m * n * c   # o and residual read, out written
    if op == "transition":
        return float(m * c * 2 * 2), 2.0 * m * c * (4 * c) * 2
    raise KeyError(op)


FUSED_CASES = (("ln_projection", 64), ("ln_projection", 128), ("output_projection", 64),
               ("output_projection", 128), ("ln_gdp", 64), ("ln_gdp", 128),
               ("trimul_epilogue", 64), ("trimul_epilogue", 128), ("transition", 64),
               ("transition", 128))


def make_fused(torch, hip, op, c, M, g):
    """Inputs for one call of `op` at width c, and the call."""
    def h(*shape, s=1.0):
        return (torch.randn(shape, generator=g, device="cuda") * s).half()

    def f(*shape, s=1.0, mean=0.0):
        return torch.randn(shape, generator=g, device="cuda") * s + mean

    if op == "ln_projection":
        x, sc, of = h(M, c), f(c, s=.1, mean=1.), f(c, s=.1)
        wT, wbT = h(512, c, s=c ** -.5), h(4, c, s=c ** -.5)
        return lambda: hip.ln_projection(x, sc, of, wT, wbT), (x, wT, wbT)
    if op == "output_projection":
        o, wT, b, r = h(M, 128), h(c, 128, s=128 ** -.5), h(c, s=.1), h(M, c)
        out = torch.empty((M, c), dtype=torch.float16, device="cuda")
        return lambda: hip.output_projection(o, wT, b, residual=r, out=out), (o, r, out)
    if op == "ln_gdp":
        x, sc, of = h(M, c), f(c, s=.1, mean=1.), f(c, s=.1)
        wpT, wgT, bp, bg = h(2 * c, c, s=c ** -.5), h(2 * c, c, s=c ** -.5), h(2 * c, s=.1), h(2 * c, s=.1)
        mask = torch.ones(M, dtype=torch.float16, device="cuda")
        return lambda: hip.ln_gdp(x, sc, of, wpT, bp, wgT, bg, mask), (x, mask)
    if op == "trimul_epilogue":
        x_cm, x = f(c, M), h(M, c)
        ins, ino, lns, lno = f(c, s=.1, mean=1.), f(c, s=.1), f(c, s=.1, mean=1.), f(c, s=.1)
        woT, bo, wgT, bg = h(c, c, s=c ** -.5), h(c, s=.1), h(c, c, s=c ** -.5), h(c, s=.1)
        out = torch.empty((M, c), dtype=torch.float16, device="cuda")
        return (lambda: hip.trimul_epilogue(x_cm, x, ins, ino, lns, lno, woT, bo, wgT, bg, out=out),
                (x_cm, x, out))
    if op == "transition":
        hd = 4 * c
        x, sc, of = h(M, c), f(c, s=.1, mean=1.), f(c, s=.1)
        w1T, b1, w2T, b2 = h(hd, c, s=c ** -.5), h(hd, s=.1), h(hd // 64, c, 64, s=hd ** -.5), h(c, s=.1)
        out = torch.empty((M, c), dtype=torch.float16, device="cuda")
        return lambda: hip.transition(x, sc, of, w1T, b1, w2T, b2, out=out), (x, out)
    raise KeyError(op)


# the reference's unfused ops and the outer product mean, on C4's pair (M = 262144 rows, c = 128)
# and on C3's residues (B = D = 384) with 16 MSA rows of 32 channels (K = 512), F = 128
OPM_B = OPM_D = 384
OPM_ROWS, OPM_C, OPM_F = 16, 32, 128
NEXT_CASES = ("layer_norm_c128", "gated_dual_proj_c128", "opm_update_f128", "opm_outer_f128")


def make_next(torch, hip, name, g):
    """Inputs and the call for one op of NEXT_CASES, with its algorithmic bytes and flops."""
    def h(*shape, s=1.0):
        return (torch.randn(shape, generator=g, device="cuda") * s).half()

    def f(*shape, s=1.0, mean=0.0):
        return torch.randn(shape, generator=g, device="cuda") * s + mean

    M, c = 262144, 128
    if name == "layer_norm_c128":
        x, sc, of = h(M, c), f(c, s=.1, mean=1.), f(c, s=.1)
        out = torch.empty_like(x)
        return lambda: hip.layer_norm(x, sc, of, 1e-5, out=out), 4.0 * M * c, 0.0
    if name == "gated_dual_proj_c128":
        n = 2 * c
        x, wp, wg, bp, bg = h(M, c), h(c, n, s=c ** -.5), h(c, n, s=c ** -.5), h(n, s=.1), h(n, s=.1)
        mask = torch.ones(M, dtype=torch.float16, device="cuda")
        out = torch.empty((M, n), dtype=torch.float16, device="cuda")
        return (lambda: hip.gated_dual_proj(x, wp, bp, wg, bg, mask, 0, out=out),
                2.0 * (M * c + M + M * n), 2.0 * M * c * 2 * n)
    B, D, K, F = OPM_B, OPM_D, OPM_ROWS * OPM_C, OPM_F
    if name == "opm_update_f128":
        lhs, t, bias = h(B, K), h(K, D, F, s=K ** -.5), f(F, s=.1)
        norm = torch.full((B, D), float(OPM_ROWS), device="cuda")
        res = h(B, D, F)
        out = torch.empty_like(res)
        byts = 2.0 * (B * K + K * D * F + 2 * B * D * F) + 4.0 * (F + B * D)
        return (lambda: hip.opm_update(lhs, t, bias, norm, res, eps=1e-3, out=out), byts,
                2.0 * B * D * F * K)
    if name == "opm_outer_f128":
        left, right, wT = h(OPM_ROWS, B, OPM_C), h(OPM_ROWS, D, 32), h(F, 32 * OPM_C, s=1 / 32)
        out = torch.empty((B, D, F), dtype=torch.float16, device="cuda")
        byts = 2.0 * (OPM_ROWS * (B * OPM_C + D * 32) + F * 32 * OPM_C + B * D * F)
        flops = 2.0 * B * D * OPM_C * 32 * (OPM_ROWS + F)
        return lambda: hip.opm_outer(left, right, wT, out=out), byts, flops
    raise KeyError(name)


def time_calls(torch, calls, iters, warmup):
    """Per-call device time (ms) of rotating calls: `iters` calls launched back to back between
    two events on the launch stream, five times. The host's launch work per call (15-25 us)
    is shorter than these kernels, so the queue stays ahead of the GPU and a call's figure is its
    kernel's duration plus the gap to the next launch; no per-call event records (which add a few
    microseconds to these 25-100 us kernels)."""
    for i in range(warmup):
        calls[i % len(calls)]()
    torch.cuda.synchronize()
    ms = []
    for _ in range(5):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(iters):
            calls[i % len(calls)]()
        e1.record()
        torch.cuda.synchronize()
        ms.append(e0.elapsed_time(e1) / iters)
    return ms


def bench_fused(torch, hip, iters, warmup):
    M = 262144
    g = torch.Generator(device="cuda")
    g.manual_seed(1)
    res = {}
    for op, c in FUSED_CASES:
        byts, flops = fused_bytes_flops(op, M, c, n=512 if op == "ln_projection" else 128,
                                        heads=4 if op == "ln_projection" else 0)
        nsets = max(3, math.ceil(3 * MALL_BYTES / byts))
        calls = [make_fused(torch, hip, op, c, M, g)[0] for _ in range(nsets)]
        ms = time_calls(torch, calls, iters, warmup)
        res["%s_c%d" % (op, c)] = roof_entry(ms, flops, byts, buffer_sets=nsets,
                                             calls_per_mean=iters)
        del calls
        torch.cuda.empty_cache()
    for name in NEXT_CASES:
        first = make_next(torch, hip, name, g)
        nsets = max(3, math.ceil(3 * MALL_BYTES / first[1]))
        calls = [first[0]] + [make_next(torch, hip, name, g)[0] for _ in range(nsets - 1)]
        ms = time_calls(torch, calls, iters, warmup)
        res[name] = roof_entry(ms, first[2], first[1], buffer_sets=nsets,
                               calls_per_mean=iters)
        del calls, first
        torch.cuda.empty_cache()
    return res


def hbm_ceiling(torch, iters=20, gib=1):
    """The attainable HBM bandwidth of plain streaming kernels on this box, for reading the fused
    ops' fractions: torch's copy (read + write), fill (write only) and row sums of an fp32 view (read
    only; the fastest torch reduction measured, within 2% of a hand-written 16-byte read loop) of
    `gib` GiB buffers, far past the 256 MB MALL; GB/s of the mean over `iters` calls (bytes moved
    by the kernel / time)."""
    n = gib << 30
    src = torch.ones(n // 2, dtype=torch.int16, device="cuda")
    dst = torch.empty_like(src)
    red = src.view(torch.float32).view(65536, -1)
    out = {}
    for name, fn, byts in (("copy", lambda: dst.copy_(src), 2 * n),
                           ("write", lambda: dst.fill_(3), n),
                           ("read", lambda: red.sum(1), n)):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(iters):
            fn()
        b.record()
        torch.cuda.synchronize()
        ms = a.elapsed_time(b) / iters
        out[name] = {"gbs": round(byts / ms / 1e6, 1), "frac": round(byts / ms / 1e6 / PEAK_GBS, 4),
                     "ms": round(ms, 4), "bytes": byts}
    del src, dst, red
    torch.cuda.empty_cache()
    return out


def cpu_baseline(torch):
    """The fp32 torch-CPU attention fwd+bwd on a row sample of C3, as TFLOP/s."""
    from oracle import cpu_ref
    rows = 128
    g = torch.Generator()
    g.manual_seed(0)
    q, k, v, dout = (torch.randn((rows, H, S, D), generator=g).half().float() for _ in range(4))
    bias = torch.randn((H, S, S), generator=g).half().float()
    kmask = torch.ones((rows, S), dtype=torch.uint8)
    scale = D ** -0.5
    cpu_ref.attention_fwd_bwd(q, k, v, bias, kmask, dout, scale)  # warm-up
    times = []
    for _ in range(5):
        t0 = time.perf_counter()
        cpu_ref.attention_fwd_bwd(q, k, v, bias, kmask, dout, scale)
        times.append(time.perf_counter() - t0)
    sec = statistics.median(times)
    flops = 14.0 * rows * H * S * S * D
    return {"value": round(flops / sec / 1e12, 5), "unit": "TFLOP/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": "%d of the 512 C3 rows, fwd+bwd by autograd, fp32 torch-CPU, median of 5 after 1 "
                      "warm-up (%.3f s per sample; the whole C3 step would take %.1f s)"
                      % (rows, sec, sec * N / rows)}


def calibration_copy(torch, mib):
    """A plain streaming kernel of known size for the HBM byte counters: bitwise_not over an
    int16 tensor of `mib` MiB reads and writes exactly that many bytes (3 calls)."""
    src = torch.ones(mib << 19, dtype=torch.int16, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.bitwise_not(src, out=dst)
    torch.cuda.synchronize()


# ---- rocprofv3 summaries -----------------------------------------------------------------

def _stage_of(kernel_name):
    for frag, stage in KERNEL_STAGES:
        if frag in kernel_name:
            return stage
    return None


def stats_summary(d):
    """Text table of every *kernel_stats.csv under d (rocprofv3 --kernel-trace --stats)."""
    files = sorted(glob.glob(os.path.join(d, "**", "*kernel_stats.csv"), recursive=True))
    if not files:
        raise SystemExit("no kernel_stats.csv under " + d)
    lines = ["%-64s %7s %12s %12s %12s %7s" % ("kernel", "calls", "avg_us", "min_us", "max_us", "pct")]
    for f in files:
        for r in csv.DictReader(open(f)):
            name = r["Name"].replace("void ", "")
            name = name if len(name) <= 64 else name[:61] + "..."
            lines.append("%-64s %7s %12.2f %12.2f %12.2f %7.2f" % (
                name, r["Calls"], float(r["AverageNs"]) / 1e3, float(r["MinNs"]) / 1e3,
                float(r["MaxNs"]) / 1e3, float(r["Percentage"])))
    return "\n".join(lines)


def _counter_means(d, counter):
    """Mean per dispatch of `counter` (summed over its instances) for each kernel name."""
    per = {}
    files = sorted(glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True))
    if not files:
        raise SystemExit("no counter_collection.csv under " + d)
    for f in files:
        for r in csv.DictReader(open(f)):
            if r["Counter_Name"] != counter:
                continue
            key = (r["Kernel_Name"], r["Dispatch_Id"])
            per[key] = per.get(key, 0.0) + float(r["Counter_Value"])
    out = {}
    for (name, _), v in per.items():
        out.setdefault(name, []).append(v)
    return {name: statistics.mean(v) for name, v in out.items()}


def traffic_summary(fetch_dir, write_dir, mib, prefix=""):
    """HBM bytes per dispatch: FETCH_SIZE and WRITE_SIZE (KiB) scaled by what the same counters
    read for the calibration copy of known size; attention stages are named prefix + stage."""
    fetch, write = _counter_means(fetch_dir, "FETCH_SIZE"), _counter_means(write_dir, "WRITE_SIZE")
    cal = [n for n in fetch if CALIBRATION_KERNEL in n]
    if not cal or not any(CALIBRATION_KERNEL in n for n in write):
        raise SystemExit("the runs hold no calibration copy (--calibration-copy)")
    known_kib = float(mib) * 1024
    f_fetch = known_kib / fetch[cal[0]]
    f_write = known_kib / next(write[n] for n in write if CALIBRATION_KERNEL in n)
    lines = ["calibration: %s over %d MiB reads FETCH_SIZE %.0f KiB and writes WRITE_SIZE %.0f KiB "
             "per dispatch; scale factors fetch %.4f, write %.4f"
             % (CALIBRATION_KERNEL, mib, fetch[cal[0]], known_kib / f_write, f_fetch, f_write)]
    for name in sorted(fetch):
        if "clk::" not in name or name not in write:
            continue
        stage = _stage_of(name)
        short = name.replace("void ", "").replace("clk::", "").split("(")[0].replace(" ", "")
        by = (fetch[name] * f_fetch + write[name] * f_write) * 1024
        lines.append("%s %s fetch_kib %.0f write_kib %.0f traffic_bytes %.0f"
                     % ("kernel" if stage else "fused", prefix + stage if stage else short,
                        fetch[name], write[name], by)
                     + ("  (%s)" % short if stage else ""))
    return "\n".join(lines)


# MI355X: 32 shader engines (8 XCDs x 4) report SQ_BUSY_CYCLES; 256 CUs x 4 SIMDs issue
SQ_ENGINES, SIMDS = 32, 1024


def derived_counters(c):
    """Utilisation ratios from one kernel's counter means (those whose counters are present):
    valu, mfma and coexec are shares of the SIMD cycles of the dispatch (SQ_BUSY_CYCLES per shader
    engine x SIMDs; SQ_ACTIVE_INST_VALU counts quad-cycles) with VALU, MFMA, or both at once busy;
    lds_conflict the share of LDS-active cycles lost to bank conflicts; wait_lds the share of wave
    cycles spent waiting on LDS; trans_per_valu transcendental VALU instructions per VALU one."""
    out = []
    busy = c.get("SQ_BUSY_CYCLES")
    if busy:
        simd = busy / SQ_ENGINES * SIMDS
        for name, key, k in (("valu", "SQ_ACTIVE_INST_VALU", 4.0), ("mfma", "SQ_VALU_MFMA_BUSY_CYCLES", 1.0),
                             ("coexec", "SQ_VALU_MFMA_COEXEC_CYCLES", 1.0)):
            if key in c:
                out.append("%s=%.3f" % (name, c[key] * k / simd))
    if c.get("SQ_LDS_IDX_ACTIVE"):
        out.append("lds_conflict=%.3f" % (c.get("SQ_LDS_BANK_CONFLICT", 0.0) / c["SQ_LDS_IDX_ACTIVE"]))
    if c.get("SQ_WAVE_CYCLES") and "SQ_WAIT_INST_LDS" in c:
        out.append("wait_lds=%.3f" % (c["SQ_WAIT_INST_LDS"] / c["SQ_WAVE_CYCLES"]))
    if c.get("SQ_INSTS_VALU") and "SQ_INSTS_VALU_TRANS_F32" in c:
        out.append("trans_per_valu=%.3f" % (c["SQ_INSTS_VALU_TRANS_F32"] / c["SQ_INSTS_VALU"]))
    return " ".join(out)


def counter_summary(dirs):
    """Mean per dispatch of every counter in one or more rocprofv3 --pmc runs, for each of the
    library's kernels (one line per kernel, counters in the order first seen), then the kernel's
    derived ratios (derived_counters) on a line of their own."""
    per, names = {}, []
    for d in dirs:
        files = sorted(glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True))
        if not files:
            raise SystemExit("no counter_collection.csv under " + d)
        for f in files:
            for r in csv.DictReader(open(f)):
                if "clk::" not in r["Kernel_Name"]:
                    continue
                c = r["Counter_Name"]
                if c not in names:
                    names.append(c)
                key = (r["Kernel_Name"], c, d, r["Dispatch_Id"])
                per[key] = per.get(key, 0.0) + float(r["Counter_Value"])
    acc = {}
    for (name, c, _, _), v in per.items():
        acc.setdefault(name, {}).setdefault(c, []).append(v)
    lines = []
    for name in sorted(acc):
        short = name.replace("void ", "").replace("clk::", "").split("(")[0].replace(" ", "")
        means = {c: statistics.mean(acc[name][c]) for c in names if c in acc[name]}
        lines.append("%s %s" % (short, " ".join("%s=%.4g" % (c, v) for c, v in means.items())))
        d = derived_counters(means)
        if d:
            lines.append("  derived %s" % d)
    return "\n".join(lines)


def load_traffic(stage):
    """HBM bytes per dispatch of `stage` (C3's, or "c2:..." / "c5:...") from the committed counter
    summaries, or None."""
    for path in (TRAFFIC_FILE, EXTRA_TRAFFIC_FILE):
        try:
            for line in open(path):
                t = line.split()
                if len(t) >= 8 and t[0] == "kernel" and t[1] == stage and t[6] == "traffic_bytes":
                    return float(t[7])
        except OSError:
            continue
    return None


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-fused", action="store_true")
    ap.add_argument("--no-packed", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the C2 and C5 configs")
    ap.add_argument("--calibration-copy", type=int, default=0, metavar="MIB")
    ap.add_argument("--only", choices=sorted(EXTRA_CONFIGS), metavar="CONFIG",
                    help="profiling: run only this extra config (c2 or c5) and print its object")
    ap.add_argument("--prefix", default="", help="stage-name prefix for --traffic-summary")
    ap.add_argument("--stats-summary", metavar="DIR")
    ap.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"))
    ap.add_argument("--counter-summary", nargs="+", metavar="DIR")
    args = ap.parse_args()
    if args.stats_summary:
        print(stats_summary(args.stats_summary))
        return
    if args.traffic_summary:
        print(traffic_summary(args.traffic_summary[0], args.traffic_summary[1], args.calibration_copy or 256,
                              args.prefix))
        return
    if args.counter_summary:
        print(counter_summary(args.counter_summary))
        return
    if args.gpus != 1:
        print("bench.py: this build runs on one GPU per box; --gpus %d is not supported "
              "(the path shards by batch rows across GPUs, which no run here exercises)" % args.gpus,
              file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    from colabfold_legacy_kernels import hip
    hip.lib()
    ev = HipEvents()
    if args.calibration_copy:
        calibration_copy(torch, args.calibration_copy)
    if args.only:
        print(json.dumps({args.only: bench_extra(torch, hip, ev, args.only, args.steps, args.warmup)}),
              flush=True)
        return
    ms_step, flops_step, kernels, ms_staged = bench_attention(torch, hip, args.steps, args.warmup, ev)
    roof = roofline_of(kernels)
    line = {
        "metric": METRIC,
        "value": round(flops_step / ms_step / 1e9, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "C3: MSA row attention with pair bias, fwd (want_lse) + bwd (want_dbias)",
                   "N_seq": N, "N_res": S, "heads": H, "head_dim": D, "flops_per_step": flops_step,
                   "frac_mfma_step": round(flops_step / ms_step / 1e9 / PEAK_TFLOPS, 4),
                   "ms_per_step_staged": round(ms_staged, 5)},
        "roofline": roof,
        "kernels": kernels,
    }
    if not args.no_extra:
        for name in EXTRA_CONFIGS:
            line[name] = bench_extra(torch, hip, ev, name, args.steps, args.warmup)
    if not args.no_packed:
        line["packed_fwd"] = bench_packed(torch, hip, args.steps, args.warmup, ev)
    if not args.no_fused:
        line["fused"] = bench_fused(torch, hip, args.steps, args.warmup)
        line["hbm_ceiling"] = hbm_ceiling(torch)
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(torch)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
