"""Pins the float64 attention oracle (oracle/attention.py) against checks that are not a
retyping of its formulas: torch's scaled_dot_product_attention, a per-element brute force,
torch float64 autograd of an independent formulation, central finite differences, closed-form
special cases and the committed golden fixtures. CPU only.
"""
import itertools
import os

import numpy as np
import pytest
import torch

from oracle import attention as ora

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def rand(seed, n=2, h=3, sq=5, sk=7, d=4, masked=0.3, amp=0.7):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((n, h, sq, d)) * amp
    k = rng.standard_normal((n, h, sk, d)) * amp
    v = rng.standard_normal((n, h, sk, d))
    bias = rng.standard_normal((h, sq, sk)) * amp
    kmask = (rng.random((n, sk)) > masked).astype(np.uint8)
    dout = rng.standard_normal((n, h, sq, d))
    return q, k, v, bias, kmask, dout


def test_forward_matches_torch_sdpa_without_bias_or_mask():
    q, k, v, _, _, _ = rand(0, n=2, h=3, sq=9, sk=11, d=8)
    bias = np.zeros((3, 9, 11))
    kmask = np.ones((2, 11), np.uint8)
    scale = 0.37
    out, lse2 = ora.attention_fwd(q, k, v, bias, kmask, scale)
    tq, tk, tv = (torch.from_numpy(x) for x in (q, k, v))
    ref = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, scale=scale).numpy()
    np.testing.assert_allclose(out, ref, rtol=1e-12, atol=1e-12)
    lse_ref = torch.logsumexp(scale * tq @ tk.transpose(-1, -2), -1).numpy() / np.log(2.0)
    np.testing.assert_allclose(lse2, lse_ref, rtol=1e-12, atol=1e-12)


def test_forward_brute_force():
    """Every output element from its definition: masked logits replaced by -1e4."""
    q, k, v, bias, kmask, _ = rand(1, n=2, h=2, sq=3, sk=5, d=3)
    scale = 0.5
    out, lse2 = ora.attention_fwd(q, k, v, bias, kmask, scale)
    for n, h, i in itertools.product(range(2), range(2), range(3)):
        logits = []
        for j in range(5):
            if kmask[n, j]:
                logits.append(scale * sum(q[n, h, i, c] * k[n, h, j, c] for c in range(3)) + bias[h, i, j])
            else:
                logits.append(-1.0e4)
        mx = max(logits)
        w = [np.exp(x - mx) for x in logits]
        z = sum(w)
        for c in range(3):
            assert abs(out[n, h, i, c] - sum(w[j] * v[n, h, j, c] for j in range(5)) / z) < 1e-12
        assert abs(lse2[n, h, i] - (np.log(z) + mx) / np.log(2.0)) < 1e-9


def torch_attention(q, k, v, bias, kmask, scale):
    """An independent torch formulation: the mask as -1e4 added via masked_fill."""
    logits = torch.matmul(q, k.transpose(-1, -2)) * scale + bias.unsqueeze(0)
    dead = torch.from_numpy(kmask == 0)[:, None, None, :].expand_as(logits)
    logits = logits.masked_fill(dead, -1.0e4)
    return torch.matmul(torch.softmax(logits, -1), v)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_backward_matches_torch_autograd(seed):
    q, k, v, bias, kmask, dout = rand(seed, n=3, h=2, sq=6, sk=9, d=5)
    kmask[1, :] = 0  # one all-masked batch row
    scale = 5 ** -0.5
    tq, tk, tv, tb = (torch.from_numpy(x).requires_grad_(True) for x in (q, k, v, bias))
    out = torch_attention(tq, tk, tv, tb, kmask, scale)
    out.backward(torch.from_numpy(dout))
    dq, dk, dv, db = ora.attention_bwd(q, k, v, bias, kmask, dout, scale)
    for got, want in ((dq, tq.grad), (dk, tk.grad), (dv, tv.grad), (db, tb.grad)):
        np.testing.assert_allclose(got, want.numpy(), rtol=1e-10, atol=1e-12)


def test_backward_finite_differences():
    q, k, v, bias, kmask, dout = rand(3, n=1, h=2, sq=3, sk=4, d=3)
    scale = 0.6
    grads = ora.attention_bwd(q, k, v, bias, kmask, dout, scale)
    base = [q, k, v, bias]
    rng = np.random.default_rng(9)
    eps = 1e-6
    for which in range(4):
        direction = rng.standard_normal(base[which].shape)
        plus = [x.copy() for x in base]
        minus = [x.copy() for x in base]
        plus[which] += eps * direction
        minus[which] -= eps * direction
        fp, _ = ora.attention_fwd(*plus, kmask, scale)
        fm, _ = ora.attention_fwd(*minus, kmask, scale)
        numeric = np.sum((fp - fm) * dout) / (2 * eps)
        analytic = np.sum(grads[which] * direction)
        assert abs(numeric - analytic) < 1e-6 * max(1.0, abs(analytic)), which


def test_one_key_gives_v_and_zero_gradients():
    q, k, v, bias, _, dout = rand(4, sk=1)
    kmask = np.ones((2, 1), np.uint8)
    out, _ = ora.attention_fwd(q, k, v, bias, kmask, 0.5)
    np.testing.assert_allclose(out, np.broadcast_to(v, out.shape), atol=1e-15)
    dq, dk, dv, db = ora.attention_bwd(q, k, v, bias, kmask, dout, 0.5)
    assert np.abs(dq).max() < 1e-14 and np.abs(dk).max() < 1e-14 and np.abs(db).max() < 1e-14
    np.testing.assert_allclose(dv[:, :, 0], dout.sum(2), atol=1e-12)


def test_all_masked_row_is_uniform():
    q, k, v, bias, kmask, dout = rand(5, n=2, sk=6)
    kmask[0, :] = 0
    out, lse2 = ora.attention_fwd(q, k, v, bias, kmask, 0.5)
    np.testing.assert_allclose(out[0], np.broadcast_to(v[0].mean(1, keepdims=True), out[0].shape), atol=1e-12)
    np.testing.assert_allclose(lse2[0], np.log2(6) + ora.MASKED_LOGIT * ora.LOG2E, rtol=1e-12)
    dq, _, _, _ = ora.attention_bwd(q, k, v, bias, kmask, dout, 0.5)
    assert np.abs(dq[0]).max() == 0.0


def test_packed_layout_indexing():
    """unpack reads slot g of p[X,Y,G,H,D] for batch row n at position s, rows or columns."""
    rng = np.random.default_rng(6)
    X, Y, G, H, D = 3, 4, 4, 2, 5
    p = rng.standard_normal((X, Y, G, H, D))
    for column in (False, True):
        q, k, v, g = ora.unpack(p, column)
        for n, h, s, d in itertools.product(range(Y if column else X), range(H), range(X if column else Y), range(D)):
            x, y = (s, n) if column else (n, s)
            assert q[n, h, s, d] == p[x, y, 0, h, d] and g[n, h, s, d] == p[x, y, 3, h, d]
        o = rng.standard_normal(q.shape)
        out = ora.repack_out(o, column)
        for n, h, s, d in itertools.product(range(Y if column else X), range(H), range(X if column else Y), range(D)):
            x, y = (s, n) if column else (n, s)
            assert out[x, y, h, d] == o[n, h, s, d]


def test_packed_gate_and_trim():
    rng = np.random.default_rng(7)
    X, Y, H, D = 3, 6, 2, 4
    p = rng.standard_normal((X, Y, 4, H, D))
    bias = rng.standard_normal((H, Y, Y))
    gb = rng.standard_normal((H, D)) * 0.1
    km = (rng.random((X, Y)) > 0.3).astype(np.uint8)
    km[:, 4:] = 0
    km[2] = 0
    out = ora.attention_packed(p, bias, km, gb, False)
    q, k, v, g = ora.unpack(p, False)
    o, _ = ora.attention_fwd(q, k, v, bias, km, D ** -0.5)
    want = ora.repack_out(o / (1 + np.exp(-(g + gb[None, :, None, :]))), False)
    np.testing.assert_allclose(out, want, atol=1e-14)
    lims = ora.trim_limits(km)
    brute = [max([j + 1 for j in range(Y) if km[n, j]], default=0) for n in range(X)]
    assert list(lims) == brute + [max(brute)]
    t = ora.attention_packed(p, bias, km, gb, False, lims=lims)
    assert np.abs(t[2]).max() == 0.0  # a row with no live key
    assert np.abs(t[:, lims[-1]:]).max() == 0.0  # queries past every row's live keys
    live = km.any(1)
    np.testing.assert_allclose(t[live][:, :lims[-1]], out[live][:, :lims[-1]], atol=1e-9)


def test_golden_fixtures():
    """Regression fixtures written by tests/golden/make_golden.py from this oracle."""
    f = np.load(os.path.join(GOLDEN, "attention_small.npz"))
    out, lse2 = ora.attention_fwd(f["q"], f["k"], f["v"], f["bias"], f["kmask"], float(f["scale"]))
    dq, dk, dv, db = ora.attention_bwd(f["q"], f["k"], f["v"], f["bias"], f["kmask"], f["dout"], float(f["scale"]))
    for name, got in (("out", out), ("lse2", lse2), ("dq", dq), ("dk", dk), ("dv", dv), ("dbias", db)):
        np.testing.assert_allclose(got, f[name], rtol=1e-12, atol=1e-12, err_msg=name)


def test_golden_c1_config():
    """Config C1 (fp32 MSA row forward, N_seq = N_res = 64, H = 8, D = 32, last 6 residues
    masked, sigmoid gate): inputs regenerate from the fixture's seed; outputs of rows 0..3 and
    float64 sums of the full outputs are committed."""
    f = np.load(os.path.join(GOLDEN, "c1_forward.npz"))
    q, k, v, bias, kmask, gate = c1_inputs(int(f["seed"]))
    scale = 32 ** -0.5
    out, lse2 = ora.attention_fwd(q, k, v, bias, kmask, scale)
    gated = out * (1 / (1 + np.exp(-gate)))
    np.testing.assert_allclose(gated[:4], f["gated_rows"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(lse2[:4], f["lse2_rows"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose([gated.sum(), np.abs(gated).sum(), lse2.sum()], f["sums"], rtol=1e-12)


def c1_inputs(seed):
    """C1 as [N = 64 MSA rows, H, S = 64, D] (batch B = 1 folded into N)."""
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((64, 8, 64, 32)).astype(np.float32).astype(np.float64)
    k = rng.standard_normal((64, 8, 64, 32)).astype(np.float32).astype(np.float64)
    v = rng.standard_normal((64, 8, 64, 32)).astype(np.float32).astype(np.float64)
    bias = rng.standard_normal((8, 64, 64)).astype(np.float32).astype(np.float64)
    kmask = np.ones((64, 64), np.uint8)
    kmask[:, 58:] = 0
    gate = rng.standard_normal((64, 8, 64, 32)).astype(np.float32).astype(np.float64)
    return q, k, v, bias, kmask, gate
