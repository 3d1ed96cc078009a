"""VoltaMma / VoltaMmaBwd on gfx950 against the float64 oracle, through the C ABI.

The cases follow the reference's tests/test_attn_bwd.py (base shapes 379-385, all-masked rows
175-181, every forward (D, block_q, block_k) 184-204, large amplitudes 207-221, tiny shapes
224-237, repeat determinism 240-259, the grid-order threshold 330-341, want flags 344-369),
with inputs drawn as its inputs() does (114-125).

Tolerances (fp16 I/O): the reference's relative metric rel < 0.05 everywhere, and at unit-scale
amplitudes an absolute bar beyond the half-ulp rounding of each fp16 result: outputs (out, lse)
<= 2e-3, gradients (dq, dk, dv, dbias) <= 5e-3. dq, dk, dv and dbias must also repeat
bit-for-bit (the backward has no atomics), which is stronger than the reference's bound.
"""
import numpy as np
import pytest
import torch

from conftest import record_error
from oracle import attention as ora

pytestmark = pytest.mark.gpu

OUT_ATOL = 2e-3
GRAD_ATOL = 5e-3
REL_TOL = 0.05

FWD_CONFIGS = ((8, 64, 64), (8, 64, 32), (8, 32, 32), (8, 128, 64), (8, 32, 64),
               (32, 64, 64), (32, 64, 32), (32, 32, 64), (32, 32, 32), (32, 128, 64),
               (32, 16, 64), (16, 64, 64), (16, 32, 32), (16, 64, 32), (64, 64, 64),
               (64, 32, 32), (24, 64, 32), (24, 32, 32), (48, 64, 32), (48, 32, 32),
               (96, 64, 32), (96, 32, 32))


def inputs(n, h, sq, sk, d, seed, masked_rows=0.15, qk_amp=0.5, vo_amp=0.5):
    rng = np.random.default_rng(seed)
    f16 = lambda x: np.asarray(x, np.float16)
    q = f16(rng.standard_normal((n, h, sq, d)) * qk_amp)
    k = f16(rng.standard_normal((n, h, sk, d)) * qk_amp)
    v = f16(rng.standard_normal((n, h, sk, d)) * vo_amp)
    bias = f16(rng.standard_normal((h, sq, sk)) * qk_amp)
    kmask = (rng.random((n, sk)) > masked_rows).astype(np.uint8)
    dout = f16(rng.standard_normal((n, h, sq, d)) * vo_amp)
    return q, k, v, bias, kmask, dout


def dev(*xs):
    return [torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in xs]


def host(*ts):
    torch.cuda.synchronize()
    return [t.float().cpu().numpy() for t in ts]


def run(hip, n=3, h=4, sq=96, sk=96, d=32, seed=0, bq=64, bk=32, kmask=None, qk_amp=0.5,
        vo_amp=0.5, want_lse=True, want_dbias=True):
    q, k, v, bias, km, dout = inputs(n, h, sq, sk, d, seed, qk_amp=qk_amp, vo_amp=vo_amp)
    if kmask is not None:
        km = kmask
    scale = float(d) ** -0.5
    tq, tk, tv, tb, tm, tdo = dev(q, k, v, bias, km, dout)
    out, lse = hip.attention_fwd(tq, tk, tv, tb, tm, scale, bq, bk, want_lse=True)
    dq, dk, dv, dbias = hip.attention_bwd(tq, tk, tv, tb, tm, out, tdo, lse, scale,
                                          want_dbias=want_dbias)
    got = dict(zip(("out", "lse", "dq", "dk", "dv", "dbias"), host(out, lse, dq, dk, dv, dbias)))
    ref_out, ref_lse = ora.attention_fwd(q, k, v, bias, km, scale)
    ref = dict(zip(("dq", "dk", "dv", "dbias"), ora.attention_bwd(q, k, v, bias, km, dout, scale)))
    ref["out"], ref["lse"] = ref_out, ref_lse
    return got, ref


def check(got, ref, label, absolute=True, names=("out", "lse", "dq", "dk", "dv", "dbias")):
    """rel < REL_TOL for every result and, with `absolute`, the north star's absolute bars on
    the error beyond each fp16 result's half-ulp rounding; the raw max-abs error of each result
    is recorded beside them for the session summary."""
    bad = []
    for name in names:
        raw, e, r = record_error(label, name, got[name], ref[name],
                                 fp16_out=name not in ("lse", "dbias"))
        if r >= REL_TOL:
            bad.append("%s %s rel %.2e (raw max abs %.2e)" % (label, name, r, raw))
        if absolute:
            tol = OUT_ATOL if name in ("out", "lse") else GRAD_ATOL
            if e > tol:
                bad.append("%s %s abs excess %.2e > %.0e (raw max abs %.2e)" % (label, name, e, tol, raw))
    assert not bad, "; ".join(bad)


@pytest.mark.parametrize("kw", [dict(sq=96, sk=96, d=32), dict(sq=96, sk=96, d=32, bq=64, bk=64),
                                dict(sq=64, sk=64, d=64, bk=64), dict(sq=70, sk=83, d=16),
                                dict(sq=128, sk=32, d=8, n=1, h=1), dict(sq=200, sk=208, d=32, n=2)])
def test_base_shapes(hip, kw):
    got, ref = run(hip, **kw)
    check(got, ref, str(kw))


@pytest.mark.parametrize("sk,frac", [(184, 0.0), (120, 0.03), (248, 0.05), (256, 0.2)])
def test_sparse_dead_keys(hip, sk, frac):
    """Key tiles with a few dead keys, masked inside Sk or past it (Sk % 64 = 56 leaves 8), and
    with more than the forward's LDS-store limit of 8 (a 20% mask): both ways a tile's dead
    keys take their logits."""
    rng = np.random.default_rng(sk)
    km = (rng.random((3, sk)) >= frac).astype(np.uint8)
    got, ref = run(hip, sq=96, sk=sk, kmask=km)
    check(got, ref, "sk=%d frac=%.2f" % (sk, frac))


def run_with_bias(hip, q, k, v, bias, km, dout, d, bq=64, bk=32):
    scale = float(d) ** -0.5
    tq, tk, tv, tb, tm, tdo = dev(q, k, v, bias, km, dout)
    out, lse = hip.attention_fwd(tq, tk, tv, tb, tm, scale, bq, bk, want_lse=True)
    dq, dk, dv, dbias = hip.attention_bwd(tq, tk, tv, tb, tm, out, tdo, lse, scale, want_dbias=True)
    got = dict(zip(("out", "lse", "dq", "dk", "dv", "dbias"), host(out, lse, dq, dk, dv, dbias)))
    ref_out, ref_lse = ora.attention_fwd(q, k, v, bias, km, scale)
    ref = dict(zip(("dq", "dk", "dv", "dbias"), ora.attention_bwd(q, k, v, bias, km, dout, scale)))
    ref["out"], ref["lse"] = ref_out, ref_lse
    return got, ref


@pytest.mark.parametrize("d,sk,bk,near", [(32, 256, 32, False), (32, 250, 64, False), (64, 256, 64, False),
                                          (8, 200, 32, False), (32, 256, 32, True), (96, 250, 32, True)])
def test_dead_key_tiles(hip, d, sk, bk, near):
    """Whole 64-key tiles with no live key after a live first tile (keys 64..127 and from 160 on
    masked in every row, the last tile ragged or past Sk where Sk % 64 != 0). With `near` the
    live keys' bias sits at -9992, 8 above the masked logit, where the masked keys still weigh
    e^-8 against the live ones (fp32 logits near 1e4 carry about 1e-3 of rounding)."""
    q, k, v, bias, _, dout = inputs(3, 2, 96, sk, d, 11)
    km = np.ones((3, sk), np.uint8)
    km[:, 64:128] = 0
    km[:, 160:] = 0
    if near:
        bias = np.full_like(bias, -9992.0)
    got, ref = run_with_bias(hip, q, k, v, bias, km, dout, d, bk=bk)
    check(got, ref, "dead tiles d=%d sk=%d near=%s" % (d, sk, near))


def random_case(i):
    """Seeded shape i of the sweep: a forward config of the reference's table, Sq and Sk from 1
    to 300 (so Sk % 8 and Sk % 64 take every kind of value: the bias-through-LDS path and the
    register path, whole and ragged key tiles), a masked fraction from none to nearly all, and
    n h Sq Sk bounded so the float64 oracle stays quick."""
    rng = np.random.default_rng(1000 + i)
    d, bq, bk = FWD_CONFIGS[int(rng.integers(len(FWD_CONFIGS)))]
    sq, sk = (int(x) for x in rng.integers(1, 301, size=2))
    n, h = int(rng.integers(1, 5)), int(rng.integers(1, 4))
    while n * h * sq * sk > 400_000:
        n, h = max(1, n // 2), max(1, h - 1) if n == 1 else h
        if n == 1 and h == 1:
            break
    frac = float(rng.choice([0.0, 0.05, 0.3, 0.9]))
    return dict(n=n, h=h, sq=sq, sk=sk, d=d, bq=bq, bk=bk, frac=frac, seed=2000 + i)


@pytest.mark.parametrize("i", range(24))
def test_random_shapes(hip, i):
    """A seeded sweep beyond the reference's fixed cases, against the oracle with the same bars."""
    c = random_case(i)
    rng = np.random.default_rng(c["seed"])
    km = (rng.random((c["n"], c["sk"])) >= c["frac"]).astype(np.uint8)
    got, ref = run(hip, n=c["n"], h=c["h"], sq=c["sq"], sk=c["sk"], d=c["d"], seed=c["seed"],
                   bq=c["bq"], bk=c["bk"], kmask=km)
    check(got, ref, "random %d %s" % (i, c))


@pytest.mark.parametrize("d,sk,bk", [(32, 96, 32), (32, 40, 32), (32, 200, 64), (8, 130, 32),
                                     (64, 136, 64), (96, 100, 32)])
def test_all_masked_row(hip, d, sk, bk):
    """A batch element with every key masked: a uniform softmax, finite lse, zero dS. The
    forward takes such a row's closed form (the mean of its V rows) once its first key tile
    shows no live key and the rest of its mask none either; Sk <= 64 has only that tile."""
    km = np.ones((3, sk), np.uint8)
    km[1, :] = 0
    km[2, 70:] = 0  # a live first tile, dead keys after it: the tile loop
    got, ref = run(hip, sk=sk, d=d, bk=bk, kmask=km)
    check(got, ref, "all-masked d=%d sk=%d" % (d, sk))
    # the closed form: out = mean of v, lse2 = log2(Sk) - 1e4 log2(e)
    lse_row = got["lse"][1]
    assert np.allclose(lse_row, np.log2(sk) + ora.MASKED_LOGIT * ora.LOG2E, atol=2e-3)


@pytest.mark.parametrize("d,bq,bk", FWD_CONFIGS)
def test_every_forward_config(hip, d, bq, bk):
    got, ref = run(hip, n=2, h=2, sq=130, sk=130, d=d, bq=bq, bk=bk)
    check(got, ref, "D=%d bq=%d bk=%d" % (d, bq, bk))


@pytest.mark.parametrize("qk,vo", [(0.5, 32.0), (0.5, 90.0), (16.0, 0.5), (32.0, 0.5)])
def test_large_amplitudes(hip, qk, vo):
    got, ref = run(hip, n=2, h=2, d=64, bk=64, qk_amp=qk, vo_amp=vo)
    check(got, ref, "qk x%g vo x%g" % (qk, vo), absolute=False)


@pytest.mark.parametrize("sq,sk,d", [(1, 1, 16), (1, 4, 16), (7, 13, 16), (33, 1, 32), (3, 96, 8)])
def test_tiny_shapes(hip, sq, sk, d):
    got, ref = run(hip, n=2, h=2, sq=sq, sk=sk, d=d)
    check(got, ref, "sq=%d sk=%d d=%d" % (sq, sk, d))


@pytest.mark.parametrize("sq,sk,d", [(96, 96, 32), (384, 384, 32), (70, 83, 16), (130, 130, 64)])
def test_masked_key_rows_do_not_matter(hip, sq, sk, d):
    """A masked key's logit is the masked logit whatever its K row (volta_attn.h:9-14), and its
    dS is 0: K rows of masked keys filled with large values (+-3e4) give out, lse, dq, dv and
    dbias bit-identical to zero rows, and dK identical. The forward and dQ kernels load K tiles
    straight into LDS at D <= 32 and zero the masked rows there; a missed row would put
    q.k scale + bias in place of the masked logit."""
    n, h = 2, 3
    q, k, v, bias, km, dout = inputs(n, h, sq, sk, d, seed=11, masked_rows=0.3)
    assert (km == 0).any() and (km != 0).any()
    rng = np.random.default_rng(12)
    dead = (km == 0)[:, None, :, None]
    k_zero = np.where(dead, np.float16(0), k).astype(np.float16)
    big = (np.sign(rng.standard_normal(k.shape)) * 3e4).astype(np.float16)
    k_big = np.where(dead, big, k).astype(np.float16)
    scale = float(d) ** -0.5
    res = []
    for kk in (k_zero, k_big):
        tq, tk, tv, tb, tm, tdo = dev(q, kk, v, bias, km, dout)
        out, lse = hip.attention_fwd(tq, tk, tv, tb, tm, scale, 64, 64 if d == 64 else 32)
        res.append(host(out, lse, *hip.attention_bwd(tq, tk, tv, tb, tm, out, tdo, lse, scale)))
    for name, x, y in zip(("out", "lse", "dq", "dk", "dv", "dbias"), *res):
        assert np.isfinite(y).all(), name + " not finite with large masked K rows"
        assert np.array_equal(x, y), name + " depends on the K rows of masked keys"


@pytest.mark.parametrize("n", [63, 64, 96])
def test_batch_sizes(hip, n):
    got, ref = run(hip, n=n, h=2, sq=64, sk=64, d=32)
    check(got, ref, "n=%d" % n)


@pytest.mark.parametrize("n,h,s,registers", [(512, 8, 96, 1), (128, 16, 128, 1), (96, 4, 200, 1),
                                              (64, 4, 300, 1), (256, 1, 416, 0), (256, 1, 448, 0)])
def test_multi_pass_dkdv(hip, n, h, s, registers):
    """Shapes whose dK/dV workgroups take several passes over batch rows, so the row cursors
    roll over, the next row's K/V prefetch is used and the dBias partial accumulates across rows:
    in registers (Sq <= 384 at D = 32: 96 with a ragged tile count, 128, 200, whose query
    tiles stop inside a 64-query step, and 300, the twelve-wave kernel with padded tiles and a
    ragged last chunk) or in LDS across row groups (416, 448). The results must also repeat bit
    for bit."""
    plan = hip.attention_bwd_plan(n, h, s, s, 32)
    assert plan["passes"] > 1 and plan["registers"] == registers, plan
    got, ref = run(hip, n=n, h=h, sq=s, sk=s, d=32, seed=3)
    check(got, ref, "multi-pass n=%d h=%d s=%d" % (n, h, s))
    q, k, v, bias, km, dout = inputs(n, h, s, s, 32, 3)
    scale = 32.0 ** -0.5
    tq, tk, tv, tb, tm, tdo = dev(q, k, v, bias, km, dout)
    out, lse = hip.attention_fwd(tq, tk, tv, tb, tm, scale)
    a = host(*hip.attention_bwd(tq, tk, tv, tb, tm, out, tdo, lse, scale))
    b = host(*hip.attention_bwd(tq, tk, tv, tb, tm, out, tdo, lse, scale))
    for name, x, y in zip(("dq", "dk", "dv", "dbias"), a, b):
        assert np.array_equal(x, y), name + " differs between identical calls"


@pytest.mark.parametrize("n,h,sq,sk,d", [(2, 2, 768, 768, 32), (2, 2, 1024, 1024, 32),
                                         (3, 2, 520, 200, 32), (2, 2, 544, 544, 64),
                                         (2, 1, 1000, 700, 96)])
def test_long_sequences_with_dbias(hip, n, h, sq, sk, d):
    """Sq past what one LDS-resident dBias partial holds (the reference's backward runs any Sq,
    cuda/volta_mma_attn_bwd.cu:336-343): the dK/dV kernel splits the queries into windows and
    sums their dK/dV in window order. Against the oracle, bit-exact on repeat, and dk/dv
    unchanged without want_dbias."""
    plan = hip.attention_bwd_plan(n, h, sq, sk, d)
    assert plan["windows"] > 1, plan
    got, ref = run(hip, n=n, h=h, sq=sq, sk=sk, d=d, seed=4, bk=64 if d == 64 else 32)
    check(got, ref, "long n=%d h=%d sq=%d sk=%d d=%d" % (n, h, sq, sk, d))
    q, k, v, bias, km, dout = inputs(n, h, sq, sk, d, 4)
    scale = float(d) ** -0.5
    tq, tk, tv, tb, tm, tdo = dev(q, k, v, bias, km, dout)
    out, lse = hip.attention_fwd(tq, tk, tv, tb, tm, scale, 64, 64 if d == 64 else 32)
    a = host(*hip.attention_bwd(tq, tk, tv, tb, tm, out, tdo, lse, scale))
    b = host(*hip.attention_bwd(tq, tk, tv, tb, tm, out, tdo, lse, scale))
    off = host(*hip.attention_bwd(tq, tk, tv, tb, tm, out, tdo, lse, scale, want_dbias=False))
    for name, x, y, z in zip(("dq", "dk", "dv", "dbias"), a, b, off):
        assert np.array_equal(x, y), name + " differs between identical calls"
        if name != "dbias":
            assert np.array_equal(x, z), name + " changed when want_dbias was off"
    assert np.abs(off[3]).max() == 0.0


@pytest.mark.parametrize("sq,sk", [(120, 100), (129, 250), (256, 256), (257, 130), (384, 70)])
def test_register_kernels_want_dbias(hip, sq, sk):
    """The register dK/dV kernels (eight waves for Sq <= 128, sixteen for Sq <= 256, twelve for
    Sq <= 384) with and without their dBias partial: dq, dk and dv are the same bits either way,
    the dbias output is zero without want_dbias, and with it the results meet the oracle."""
    plan = hip.attention_bwd_plan(2, 2, sq, sk, 32)
    assert plan["registers"] == 1, plan
    got, ref = run(hip, n=2, h=2, sq=sq, sk=sk, d=32, seed=5)
    check(got, ref, "register sq=%d sk=%d" % (sq, sk))
    q, k, v, bias, km, dout = inputs(2, 2, sq, sk, 32, 5)
    scale = 32.0 ** -0.5
    tq, tk, tv, tb, tm, tdo = dev(q, k, v, bias, km, dout)
    out, lse = hip.attention_fwd(tq, tk, tv, tb, tm, scale)
    on = host(*hip.attention_bwd(tq, tk, tv, tb, tm, out, tdo, lse, scale))
    off = host(*hip.attention_bwd(tq, tk, tv, tb, tm, out, tdo, lse, scale, want_dbias=False))
    for name, x, y in zip(("dq", "dk", "dv"), on[:3], off[:3]):
        assert np.array_equal(x, y), name + " changed when want_dbias was off"
    assert np.abs(off[3]).max() == 0.0


def test_repeat_bit_exact(hip):
    q, k, v, bias, km, dout = inputs(3, 4, 96, 96, 32, 0)
    scale = 32.0 ** -0.5
    tq, tk, tv, tb, tm, tdo = dev(q, k, v, bias, km, dout)
    out, lse = hip.attention_fwd(tq, tk, tv, tb, tm, scale)
    a = host(*hip.attention_bwd(tq, tk, tv, tb, tm, out, tdo, lse, scale))
    b = host(*hip.attention_bwd(tq, tk, tv, tb, tm, out, tdo, lse, scale))
    for name, x, y in zip(("dq", "dk", "dv", "dbias"), a, b):
        assert np.array_equal(x, y), name + " differs between identical calls"


def test_want_flags(hip):
    """want_lse and want_dbias only drop results (tests/test_attn_bwd.py:344-369)."""
    q, k, v, bias, km, dout = inputs(2, 2, 96, 96, 32, 0)
    scale = 32.0 ** -0.5
    tq, tk, tv, tb, tm, tdo = dev(q, k, v, bias, km, dout)
    out, lse = hip.attention_fwd(tq, tk, tv, tb, tm, scale)
    lse_one = torch.full((1,), 7.0, dtype=torch.float32, device="cuda")
    out_off, lse_off = hip.attention_fwd(tq, tk, tv, tb, tm, scale, want_lse=False, lse=lse_one)
    on = host(*hip.attention_bwd(tq, tk, tv, tb, tm, out, tdo, lse, scale))
    off = host(*hip.attention_bwd(tq, tk, tv, tb, tm, out, tdo, lse, scale, want_dbias=False))
    o1, o2, l1 = host(out, out_off, lse_off)
    assert np.array_equal(o1, o2), "out changed when want_lse was off"
    assert l1[0] == 7.0, "the one-element lse was written without want_lse"
    for name, x, y in zip(("dq", "dk", "dv"), on[:3], off[:3]):
        assert np.array_equal(x, y), name + " changed when want_dbias was off"
    assert np.abs(off[3]).max() == 0.0, "dbias was written although want_dbias was off"


@pytest.mark.parametrize("n,sq,sk", [(2, 0, 40), (0, 24, 40), (2, 24, 0)])
def test_empty_problems(hip, n, sq, sk):
    """No query, no row or no key: every gradient is an empty sum, written as zeros over the
    NaN the results held before the call."""
    h, d = 2, 32
    q = torch.zeros((n, h, sq, d), dtype=torch.float16, device="cuda")
    k = torch.zeros((n, h, sk, d), dtype=torch.float16, device="cuda")
    bias = torch.zeros((h, sq, sk), dtype=torch.float16, device="cuda")
    kmask = torch.ones((n, sk), dtype=torch.uint8, device="cuda")
    lse = torch.zeros((n, h, sq), dtype=torch.float32, device="cuda")
    grads = (torch.full_like(q, float("nan")), torch.full_like(k, float("nan")),
             torch.full_like(k, float("nan")), torch.full(bias.shape, float("nan"), device="cuda"))
    hip.attention_bwd(q, k, k, bias, kmask, q, q, lse, d ** -0.5, grads=grads)
    for name, t in zip(("dq", "dk", "dv", "dbias"), host(*grads)):
        assert t.size == 0 or np.abs(t).max() == 0.0, name
