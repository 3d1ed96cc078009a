"""The BASELINE.json configurations run through the C ABI at their own shapes, against the float64
oracle on the same fp16-rounded inputs.

  C1  the CPU config (fp32 MSA row forward, 64 x 64, H = 8, D = 32, last 6 residues masked,
      sigmoid gate) rounded to fp16 and run as the gated packed forward (VoltaMmaPacked, G = 4);
      checked against the oracle on the rounded inputs, and loosely against the committed
      fixture tests/golden/c1_forward.npz, which the oracle wrote from the unrounded inputs.
  C2  triangle attention forward + backward, N_res = 256: q, k, v projected from a pair
      z [256, 256, 128] by 1/sqrt(128)-scaled weights, bias ~ N(0, 0.5), 13 residues (5%)
      padded, kmask = res_mask (x) res_mask (so 13 batch rows are fully masked), dOut ~ N(0, 1).
  C3  the headline: MSA row attention [512, 8, 384, 32], all ~ N(0, 1), all-ones kmask,
      (block_q, block_k) = (64, 32), want_lse and want_dbias, dbias over all 512 rows.
  C5  triangle attention forward only, [1024, 4, 1024, 32], 8% of residues masked, want_lse
      off with a one-element lse that must stay untouched; a sample of batch rows (first,
      last, fully masked and random ones) is checked, since a row's output depends on that
      row alone.

Tolerances are the north star's (fp16 I/O): abs error beyond each fp16 result's half-ulp
rounding <= 2e-3 on outputs (out, lse) and <= 5e-3 on gradients (dq, dk, dv, dbias), plus the
reference tests' relative metric < 0.05; the raw max-abs error of every result is printed in
the session summary.
"""
import os

import numpy as np
import pytest
import torch

from conftest import record_error
from oracle import attention as ora
from test_attention_gpu import GRAD_ATOL, OUT_ATOL, REL_TOL, check, dev, host

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def normal16(rng, *shape, s=1.0):
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(s)).astype(np.float16)


def residue_mask(rng, n, frac):
    dead = rng.choice(n, size=int(round(frac * n)), replace=False)
    live = np.ones(n, np.uint8)
    live[dead] = 0
    return live


def fwd_bwd(hip, q, k, v, bias, km, dout, scale, rows=32):
    tq, tk, tv, tb, tm, tdo = dev(q, k, v, bias, km, dout)
    out, lse = hip.attention_fwd(tq, tk, tv, tb, tm, scale, 64, 32, want_lse=True)
    dq, dk, dv, dbias = hip.attention_bwd(tq, tk, tv, tb, tm, out, tdo, lse, scale, want_dbias=True)
    got = dict(zip(("out", "lse", "dq", "dk", "dv", "dbias"), host(out, lse, dq, dk, dv, dbias)))
    del tq, tk, tv, tb, tm, tdo, out, lse, dq, dk, dv, dbias
    torch.cuda.empty_cache()
    ref = {}
    ref["out"], ref["lse"] = ora.attention_fwd_chunked(q, k, v, bias, km, scale, rows=rows)
    ref["dq"], ref["dk"], ref["dv"], ref["dbias"] = ora.attention_bwd_chunked(
        q, k, v, bias, km, dout, scale, rows=rows)
    return got, ref


def test_c3_headline(hip):
    """C3 exactly as bench.py times it: the planner's multi-pass dK/dV plan, the straight-line
    bias path, twelve 32-query tiles per row and dbias reduced over all 512 rows."""
    rng = np.random.default_rng(0)
    n, h, s, d = 512, 8, 384, 32
    q, k, v, dout = (normal16(rng, n, h, s, d) for _ in range(4))
    bias = normal16(rng, h, s, s)
    km = np.ones((n, s), np.uint8)
    print("C3 [512, 8, 384, 32] forward + backward", flush=True)
    got, ref = fwd_bwd(hip, q, k, v, bias, km, dout, d ** -0.5)
    check(got, ref, "C3")


def test_c2_triangle(hip):
    """C2: q, k, v projected from the pair, padded residues on both axes (fully masked rows)."""
    rng = np.random.default_rng(2)
    nres, c, h, d = 256, 128, 4, 32
    z = rng.standard_normal((nres, nres, c), dtype=np.float32)
    w = [(rng.standard_normal((c, h * d), dtype=np.float32) * np.float32(c ** -0.5)) for _ in range(3)]
    # [i, j, h, d] -> [N = i, H, S = j, D]
    q, k, v = (np.ascontiguousarray((z.reshape(-1, c) @ wi).astype(np.float16)
                                    .reshape(nres, nres, h, d).transpose(0, 2, 1, 3)) for wi in w)
    bias = normal16(rng, h, nres, nres, s=0.5)
    res = residue_mask(rng, nres, 0.05)
    km = np.ascontiguousarray(res[:, None] * res[None, :])
    dout = normal16(rng, nres, h, nres, d)
    assert (km.sum(1) == 0).sum() == 13
    print("C2 [256, 4, 256, 32] forward + backward", flush=True)
    got, ref = fwd_bwd(hip, q, k, v, bias, km, dout, d ** -0.5)
    check(got, ref, "C2")


def test_c5_forward_sampled_rows(hip):
    """C5: forward only, want_lse off with a one-element lse (left at its sentinel)."""
    rng = np.random.default_rng(5)
    n, h, s, d = 1024, 4, 1024, 32
    q, k, v = (normal16(rng, n, h, s, d) for _ in range(3))
    bias = normal16(rng, h, s, s)
    res = residue_mask(rng, s, 0.08)
    km = np.ascontiguousarray(res[:, None] * res[None, :])
    scale = d ** -0.5
    print("C5 [1024, 4, 1024, 32] forward, want_lse off", flush=True)
    tq, tk, tv, tb, tm = dev(q, k, v, bias, km)
    lse_one = torch.full((1,), -3.5, dtype=torch.float32, device="cuda")
    out, lse = hip.attention_fwd(tq, tk, tv, tb, tm, scale, 64, 32, want_lse=False, lse=lse_one)
    got_out, got_lse = host(out, lse)
    assert got_lse.shape == (1,) and got_lse[0] == -3.5, "the one-element lse was written"
    dead = np.flatnonzero(res == 0)
    rows = sorted(set([0, n - 1, int(dead[0]), int(dead[-1])] +
                      rng.choice(n, size=20, replace=False).tolist()))
    ref_out, _ = ora.attention_fwd(q[rows], k[rows], v[rows], bias, km[rows], scale)
    check({"out": got_out[rows]}, {"out": ref_out}, "C5 rows", names=("out",))
    # every output is finite, masked rows included
    assert np.isfinite(got_out).all()


def test_c1_packed_gated(hip):
    """C1's workload (biased, gated, last 6 residues masked) through VoltaMmaPacked."""
    from test_oracle_attention import c1_inputs
    f = np.load(os.path.join(GOLDEN, "c1_forward.npz"))
    q, k, v, bias, km, gate = c1_inputs(int(f["seed"]))
    # rows attend along Y with batch X: p[x, y, slot, h, d] = slot[n = x, h, s = y, d]
    p = np.stack([a.transpose(0, 2, 1, 3) for a in (q, k, v, gate)], axis=2).astype(np.float16)
    bias16 = bias.astype(np.float16)
    gate_bias = np.zeros((8, 32), np.float16)
    scale = 32 ** -0.5
    tp, tb, tm, tg = dev(p, bias16, km, gate_bias)
    out = host(hip.attention_packed(tp, tb, tm, tg, scale, 64, 32, column=False))[0]
    want = ora.attention_packed(p, bias16, km, gate_bias, False, scale)
    check({"out": out}, {"out": want}, "C1 packed", names=("out",))
    # the fixture's rows 0..3, from the unrounded fp32 inputs: the fp16 input rounding alone
    # moves them by 9e-4
    fixture = f["gated_rows"].transpose(0, 2, 1, 3)  # [N, H, S, D] -> [X, Y, H, D]
    raw, _, _ = record_error("C1 vs fixture", "out", out[:4], fixture, fp16_out=False)
    assert raw < 5e-3, "C1 rows 0..3 differ from the fixture by %.2e" % raw
