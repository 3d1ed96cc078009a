#!/usr/bin/env python3
"""Benchmark of the ColabFold legacy-kernel hot path on one MI355X (gfx950).

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-fused]

A step is one attention forward + backward of BASELINE config C3 (MSA row attention with pair
bias, fp16: N_seq = 512 rows, N_res = 384, H = 8, D = 32): VoltaMma(want_lse) then
VoltaMmaBwd(want_dbias), through the library's C ABI on the current stream, inputs already in
HBM. value is the step's algorithmic TFLOP/s (14 u flops, u = N H S^2 D, as BASELINE counts
it: the backward's recompute of S included). Per-kernel durations come from HIP events the
library records at its kernel boundaries during the timed steps (clk_set_stage_events); the
roofline object is the dominant kernel's. The fused LayerNorm projections (config C4,
M = 262144 rows, c = 64 and 128) are timed separately, rotating enough buffer sets that no call
finds its inputs in the 256 MB Infinity Cache, and reported under "fused". cpu_baseline is the
fp32 torch-CPU restatement of the reference tests' jnp attention (oracle/cpu_ref.py; jax is not
installed) on a bounded row sample of the same workload, on this box's host cores.

One GPU per box here: --gpus above 1 exits with a message.
"""
import argparse
import ctypes
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

N, H, S, D = 512, 8, 384, 32


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


def attention_bytes():
    """Algorithmic HBM bytes per launch (each tensor read or written once)."""
    t = N * H * S * D * 2          # one fp16 [N,H,S,D] tensor
    row = N * H * S * 4            # one fp32 [N,H,S] row statistic
    bias = H * S * S * 2
    km = N * S
    return t, row, bias, km


def bench_attention(torch, hip, steps, warmup, ev):
    u = float(N) * H * S * S * D
    scale = D ** -0.5
    g = torch.Generator(device="cuda")
    g.manual_seed(0)
    sets = []
    for _ in range(2):   # two sets: a step never finds the previous step's tensors in the MALL
        q, k, v, dout = (torch.randn((N, H, S, D), generator=g, device="cuda").half() for _ in range(4))
        bias = torch.randn((H, S, S), generator=g, device="cuda").half()
        kmask = torch.ones((N, S), dtype=torch.uint8, device="cuda")
        out = torch.empty_like(q)
        lse = torch.empty((N, H, S), dtype=torch.float32, device="cuda")
        ws = torch.empty(hip.attention_bwd_workspace(q, k), dtype=torch.uint8, device="cuda")
        sets.append((q, k, v, bias, kmask, dout, out, lse, ws))

    def step(st, fwd_ev=None, bwd_ev=None):
        q, k, v, bias, kmask, dout, out, lse, ws = st
        if fwd_ev:
            arm(hip, fwd_ev)
        hip.attention_fwd(q, k, v, bias, kmask, scale, 64, 32, True, out=out, lse=lse)
        if bwd_ev:
            arm(hip, bwd_ev)
        r = hip.attention_bwd(q, k, v, bias, kmask, out, dout, lse, scale, True, workspace=ws)
        if bwd_ev:
            disarm(hip)
        return r

    for i in range(warmup):
        step(sets[i % 2])
    torch.cuda.synchronize()
    fwd_evs = [ev.create(2) for _ in range(steps)]
    bwd_evs = [ev.create(4) for _ in range(steps)]
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for i in range(steps):
        step(sets[i % 2], fwd_evs[i], bwd_evs[i])
    stop.record()
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(stop)
    per = {"attn_fwd": [], "bwd_dq": [], "bwd_dkdv": [], "bwd_dbias": []}
    for fe, be in zip(fwd_evs, bwd_evs):
        per["attn_fwd"].append(ev.elapsed_ms(fe[0], fe[1]))
        per["bwd_dq"].append(ev.elapsed_ms(be[0], be[1]))
        per["bwd_dkdv"].append(ev.elapsed_ms(be[1], be[2]))
        per["bwd_dbias"].append(ev.elapsed_ms(be[2], be[3]))
    for e in fwd_evs + bwd_evs:
        ev.destroy(e)
    disarm(hip)

    t, row, bias_b, km = attention_bytes()
    ws_bytes = sets[0][8].numel()
    partial = max(ws_bytes - row, 0)
    algo = {  # (flops, bytes) per launch
        "attn_fwd": (4 * u, 3 * t + bias_b + km + t + row),
        "bwd_dq": (6 * u, 5 * t + row + bias_b + km + t + row),
        "bwd_dkdv": (8 * u, 4 * t + 2 * row + bias_b + km + 2 * t + partial),
        "bwd_dbias": (0.0, partial + H * S * S * 4),
    }
    kernels = {}
    for name, ds in per.items():
        ms = statistics.mean(ds)
        fl, by = algo[name]
        t_mfma = fl / (PEAK_TFLOPS * 1e12) * 1e3
        t_hbm = by / (PEAK_GBS * 1e9) * 1e3
        kernels[name] = {"ms": round(ms, 5), "tflops": round(fl / ms / 1e9, 2),
                         "gbs": round(by / ms / 1e6, 1), "bound": "mfma" if t_mfma > t_hbm else "hbm",
                         "frac_mfma": round(t_mfma / ms, 4), "frac_hbm": round(t_hbm / ms, 4),
                         "algo_flops": fl, "algo_bytes": by}
    ms_step = total_ms / steps
    return ms_step, 14 * u, kernels


def fused_cases(torch):
    """(name, c, callable factory) for the C4 fused ops at M = 262144 rows."""
    return [("ln_projection", 64), ("ln_projection", 128), ("output_projection", 64),
            ("output_projection", 128), ("ln_gdp", 64), ("ln_gdp", 128),
            ("trimul_epilogue", 64), ("trimul_epilogue", 128), ("transition", 64),
            ("transition", 128)]


def make_fused(torch, hip, op, c, M, g):
    """Inputs for one call of `op` at width c, and the call."""
    def h(*shape, s=1.0):
        return (torch.randn(shape, generator=g, device="cuda") * s).half()

    def f(*shape, s=1.0, mean=0.0):
        return torch.randn(shape, generator=g, device="cuda") * s + mean

    if op == "ln_projection":
        x, sc, of = h(M, c), f(c, s=.1, mean=1.), f(c, s=.1)
        wT, wbT = h(512, c, s=c ** -.5), h(4, c, s=c ** -.5)
        p = torch.empty((M, 512), dtype=torch.float16, device="cuda")
        bias = torch.empty((4, M), dtype=torch.float16, device="cuda")
        one = torch.zeros(1, dtype=torch.float16, device="cuda")
        bufs = [hip.buffer(t) for t in (x, sc, of, wT, wbT, one, p, bias)]
        keepalive = (x, sc, of, wT, wbT, one, p, bias)
        return lambda: hip._check(hip.lib().clk_ln_projection(hip._stream(x), *map(hip._ref, bufs), 1e-5, 512, 4, 0)), keepalive
    if op == "output_projection":
        o, wT, b, r = h(M, 128), h(c, 128, s=128 ** -.5), h(c, s=.1), h(M, c)
        one = torch.zeros(1, dtype=torch.float16, device="cuda")
        out = torch.empty((M, c), dtype=torch.float16, device="cuda")
        bufs = [hip.buffer(t) for t in (o, wT, b, r, one, out)]
        return lambda: hip._check(hip.lib().clk_output_projection(hip._stream(o), *map(hip._ref, bufs), 1, 0)), (o, wT, b, r, one, out)
    if op == "ln_gdp":
        x, sc, of = h(M, c), f(c, s=.1, mean=1.), f(c, s=.1)
        wpT, wgT, bp, bg = h(2 * c, c, s=c ** -.5), h(2 * c, c, s=c ** -.5), h(2 * c, s=.1), h(2 * c, s=.1)
        mask = torch.ones(M, dtype=torch.float16, device="cuda")
        left = torch.empty((c, M), dtype=torch.float16, device="cuda")
        right = torch.empty((c, M), dtype=torch.float16, device="cuda")
        bufs = [hip.buffer(t) for t in (x, sc, of, wpT, bp, wgT, bg, mask, left, right)]
        return lambda: hip._check(hip.lib().clk_ln_gdp(hip._stream(x), *map(hip._ref, bufs), 1e-5)), (x, sc, of, wpT, bp, wgT, bg, mask, left, right)
    if op == "trimul_epilogue":
        x_cm, x = f(c, M), h(M, c)
        ins, ino, lns, lno = f(c, s=.1, mean=1.), f(c, s=.1), f(c, s=.1, mean=1.), f(c, s=.1)
        woT, bo, wgT, bg = h(c, c, s=c ** -.5), h(c, s=.1), h(c, c, s=c ** -.5), h(c, s=.1)
        one = torch.zeros(1, dtype=torch.float16, device="cuda")
        out = torch.empty((M, c), dtype=torch.float16, device="cuda")
        bufs = [hip.buffer(t) for t in (x_cm, x, ins, ino, lns, lno, woT, bo, wgT, bg, one, out)]
        return lambda: hip._check(hip.lib().clk_trimul_epilogue(hip._stream(x), *map(hip._ref, bufs), 1e-5, 0, 0)), (x_cm, x, ins, ino, lns, lno, woT, bo, wgT, bg, one, out)
    if op == "transition":
        hd = 4 * c
        x, sc, of = h(M, c), f(c, s=.1, mean=1.), f(c, s=.1)
        w1T, b1, w2T, b2 = h(hd, c, s=c ** -.5), h(hd, s=.1), h(hd // 64, c, 64, s=hd ** -.5), h(c, s=.1)
        one = torch.zeros(1, dtype=torch.float16, device="cuda")
        out = torch.empty((M, c), dtype=torch.float16, device="cuda")
        bufs = [hip.buffer(t) for t in (x, sc, of, w1T, b1, w2T, b2, one, out)]
        return lambda: hip._check(hip.lib().clk_transition(hip._stream(x), *map(hip._ref, bufs), 1e-5, 0, 0)), (x, sc, of, w1T, b1, w2T, b2, one, out)
    raise KeyError(op)


def bench_fused(torch, hip, ev, iters=20, warmup=3):
    from oracle import fused as orf
    M = 262144
    g = torch.Generator(device="cuda")
    g.manual_seed(1)
    res = {}
    for op, c in fused_cases(torch):
        if op == "ln_projection":
            byts, flops = orf.fused_bytes_flops(op, M, c, n=512, heads=4)
        elif op == "output_projection":
            byts, flops = orf.fused_bytes_flops(op, M, c, n=128)
        else:
            byts, flops = orf.fused_bytes_flops(op, M, c)
        nsets = max(3, math.ceil(3 * MALL_BYTES / byts))
        calls = [make_fused(torch, hip, op, c, M, g) for _ in range(nsets)]
        for i in range(warmup):
            calls[i % nsets][0]()
        torch.cuda.synchronize()
        evs = [ev.create(2) for _ in range(iters)]
        for i in range(iters):
            arm(hip, evs[i])
            calls[i % nsets][0]()
        disarm(hip)
        torch.cuda.synchronize()
        ms = statistics.median(ev.elapsed_ms(e[0], e[1]) for e in evs)
        for e in evs:
            ev.destroy(e)
        t_hbm = byts / (PEAK_GBS * 1e9) * 1e3
        t_mfma = flops / (PEAK_TFLOPS * 1e12) * 1e3
        bound = "mfma" if t_mfma > t_hbm else "hbm"
        res["%s_c%d" % (op, c)] = {
            "ms": round(ms, 5), "gbs": round(byts / ms / 1e6, 1), "tflops": round(flops / ms / 1e9, 2),
            "bound": bound, "frac": round(max(t_hbm, t_mfma) / ms, 4), "frac_hbm": round(t_hbm / ms, 4),
            "algo_bytes": byts, "algo_flops": flops, "buffer_sets": nsets}
        del calls
        torch.cuda.empty_cache()
    return res


def cpu_baseline(torch):
    """The fp32 torch-CPU attention fwd+bwd on a row sample of C3, as TFLOP/s."""
    from oracle import cpu_ref
    rows = 32
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
            "sample": "%d of the 512 C3 rows, fwd+bwd by autograd, fp32, median of 5 after 1 warm-up "
                      "(%.3f s per sample; whole C3 step would take %.1f s)" % (rows, sec, sec * N / rows)}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-fused", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build runs on one GPU per box; --gpus %d is not supported "
              "(the path shards by batch rows; see the design notes)" % args.gpus, file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    from colabfold_legacy_kernels import hip
    hip.lib()
    ev = HipEvents()
    ms_step, flops_step, kernels = bench_attention(torch, hip, args.steps, args.warmup, ev)
    dom = max(kernels, key=lambda k: kernels[k]["ms"])
    kd = kernels[dom]
    if kd["bound"] == "mfma":
        roof = {"bound": "mfma", "achieved": kd["tflops"], "peak": PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(kd["tflops"] / PEAK_TFLOPS, 4)}
    else:
        roof = {"bound": "hbm", "achieved": kd["gbs"], "peak": PEAK_GBS, "unit": "GB/s",
                "frac": round(kd["gbs"] / PEAK_GBS, 4)}
    roof["kernel"] = dom
    roof["traffic"] = None
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
                   "frac_mfma_step": round(flops_step / ms_step / 1e9 / PEAK_TFLOPS, 4)},
        "roofline": roof,
        "kernels": kernels,
    }
    if not args.no_fused:
        line["fused"] = bench_fused(torch, hip, ev)
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(torch)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
