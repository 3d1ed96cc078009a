"""Writes the golden fixtures in this directory from the float64 oracle (run from the repo root):

  python tests/golden/make_golden.py

attention_small.npz  a tiny masked, biased attention case (one all-masked row) with its forward
                     and backward results
c1_forward.npz       config C1's seed, its gated outputs and lse for rows 0..3 and float64 sums
                     of the full results (the inputs regenerate from the seed)
fused_small.npz      each fused op on tiny inputs, with keep tiles of every kind

The reference commits no fixtures (its tests draw inputs at run time), so these pin the oracle
against later edits of itself; what pins it to the mathematics is in tests/test_oracle_*.py.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
sys.path.insert(0, os.path.dirname(HERE))

from oracle import attention as ora  # noqa: E402
from oracle import fused as orf  # noqa: E402
from test_oracle_attention import c1_inputs  # noqa: E402
from test_oracle_fused import fused_inputs  # noqa: E402


def attention_small():
    rng = np.random.default_rng(20260)
    n, h, sq, sk, d = 3, 2, 7, 13, 8
    f16 = lambda x: x.astype(np.float16).astype(np.float64)
    q = f16(rng.standard_normal((n, h, sq, d)) * 0.5)
    k = f16(rng.standard_normal((n, h, sk, d)) * 0.5)
    v = f16(rng.standard_normal((n, h, sk, d)) * 0.5)
    bias = f16(rng.standard_normal((h, sq, sk)) * 0.5)
    kmask = (rng.random((n, sk)) > 0.2).astype(np.uint8)
    kmask[2] = 0
    dout = f16(rng.standard_normal((n, h, sq, d)) * 0.5)
    scale = d ** -0.5
    out, lse2 = ora.attention_fwd(q, k, v, bias, kmask, scale)
    dq, dk, dv, db = ora.attention_bwd(q, k, v, bias, kmask, dout, scale)
    np.savez_compressed(os.path.join(HERE, "attention_small.npz"), q=q, k=k, v=v, bias=bias,
                        kmask=kmask, dout=dout, scale=scale, out=out, lse2=lse2, dq=dq, dk=dk,
                        dv=dv, dbias=db)


def c1_forward():
    seed = 11
    q, k, v, bias, kmask, gate = c1_inputs(seed)
    out, lse2 = ora.attention_fwd(q, k, v, bias, kmask, 32 ** -0.5)
    gated = out * (1 / (1 + np.exp(-gate)))
    np.savez_compressed(os.path.join(HERE, "c1_forward.npz"), seed=seed, gated_rows=gated[:4],
                        lse2_rows=lse2[:4], sums=np.array([gated.sum(), np.abs(gated).sum(), lse2.sum()]))


def fused_small():
    inp = fused_inputs(31)
    res = {}
    l, r = orf.ln_gdp(inp["x"], inp["sc"], inp["of"], inp["wpT"], inp["bp"], inp["wgT"], inp["bg"],
                      inp["mask"], 1e-5)
    res["gdp_left"], res["gdp_right"] = l, r
    res["epi"] = orf.trimul_epilogue(inp["x_cm"], inp["x"], inp["sc"], inp["of"], inp["lsc"], inp["lof"],
                                     inp["woT"], inp["bo"], inp["wgT2"], inp["bg2"], inp["keep"], 1e-5, False)
    p, b = orf.ln_projection(inp["x"], inp["sc"], inp["of"], inp["wT"], inp["wbT"], inp["keep"], 1e-5)
    res["proj_p"], res["proj_bias"] = p, b
    res["outp"] = orf.output_projection(inp["o"], inp["woT"], inp["bo"], inp["res"], inp["keep"])
    res["trans"] = orf.transition(inp["x"], inp["sc"], inp["of"], inp["w1T"], inp["b1"], inp["w2T"],
                                  inp["b2"], inp["keep"], 1e-5, True)
    np.savez_compressed(os.path.join(HERE, "fused_small.npz"), seed=31, **res)


if __name__ == "__main__":
    attention_small()
    c1_forward()
    fused_small()
    print("fixtures written to", HERE)
