"""clk_attention_bwd_noalloc, the backward entry point that allocates nothing (its scratch is the
library's static per-GPU array), against clk_attention_bwd on the same inputs, through the C ABI.
Both run the same kernels on the same plan, so the results must agree bit for bit, which is
stronger than the north star's gradient tolerance. Calls come in a row with different shapes
(the second smaller), as the shared scratch keeps the last call's contents."""
import ctypes

import numpy as np
import pytest
import torch

from test_attention_gpu import dev, host, inputs


def _grads(q, k, bias):
    nan = float("nan")
    return (torch.full_like(q, nan), torch.full_like(k, nan), torch.full_like(k, nan),
            torch.full(bias.shape, nan, dtype=torch.float32, device=q.device))


def _compare(hip, n, h, sq, sk, d, seed, want_dbias=True):
    q, k, v, bias, km, dout = inputs(n, h, sq, sk, d, seed)
    scale = float(d) ** -0.5
    tq, tk, tv, tb, tm, tdo = dev(q, k, v, bias, km, dout)
    out, lse = hip.attention_fwd(tq, tk, tv, tb, tm, scale, 64, 64 if d == 64 else 32)
    want = host(*hip.attention_bwd(tq, tk, tv, tb, tm, out, tdo, lse, scale, want_dbias,
                                   grads=_grads(tq, tk, tb)))
    got = host(*hip.attention_bwd_noalloc(tq, tk, tv, tb, tm, out, tdo, lse, scale, want_dbias,
                                          grads=_grads(tq, tk, tb)))
    for name, x, y in zip(("dq", "dk", "dv", "dbias"), got, want):
        assert np.array_equal(x, y), "%s differs from clk_attention_bwd at %s" % (
            name, (n, h, sq, sk, d))


@pytest.mark.gpu
def test_noalloc_matches_workspace_entry_point(hip):
    print("noalloc: C3 [512, 8, 384, 32], then [3, 4, 96, 80, 32]", flush=True)
    _compare(hip, 512, 8, 384, 384, 32, seed=7)
    _compare(hip, 3, 4, 96, 80, 32, seed=8)


@pytest.mark.gpu
def test_noalloc_query_windows_and_flags(hip):
    """A plan with query windows (fp32 dK/dV window sums in the scratch), then a smaller call
    without want_dbias, then a D = 64 one."""
    print("noalloc: [2, 2, 1024, 1024, 32], [2, 2, 200, 100, 32] no dbias, [2, 2, 130, 130, 64]",
          flush=True)
    assert hip.attention_bwd_plan(2, 2, 1024, 1024, 32)["windows"] > 1
    _compare(hip, 2, 2, 1024, 1024, 32, seed=9)
    _compare(hip, 2, 2, 200, 100, 32, seed=10, want_dbias=False)
    _compare(hip, 2, 2, 130, 130, 64, seed=11)


def test_noalloc_rejects_shapes_beyond_its_scratch():
    """Shapes whose scratch exceeds the static array are refused before any launch (CPU)."""
    from colabfold_legacy_kernels import hip
    lib = hip.lib()
    fake = 0x100000  # never dereferenced: the call fails validation first
    keep = []

    def buf(dtype, *dims):
        arr = (ctypes.c_int64 * len(dims))(*dims)
        b = hip.Buffer(fake, dtype, len(dims), arr)
        keep.append((arr, b))
        return ctypes.byref(b)

    n, h, s, d = 8192, 8, 384, 32
    t = (n, h, s, d)
    args = [buf(10, *t), buf(10, *t), buf(10, *t), buf(10, h, s, s), buf(6, n, s), buf(10, *t),
            buf(10, *t), buf(11, n, h, s), buf(10, *t), buf(10, *t), buf(10, *t), buf(11, h, s, s)]
    st = lib.clk_attention_bwd_noalloc(None, 0, *args, ctypes.c_float(0.1), 1)
    assert st == hip.INVALID_ARGUMENT
    msg = lib.clk_last_error().decode()
    assert "static scratch holds %d" % lib.clk_attention_bwd_noalloc_scratch_size() in msg, msg
