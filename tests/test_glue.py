"""The caller glue on the CPU: the weight re-layouts element by element against their
definitions (cuda/volta_fused_ffi.h:42-43, 135-136, 178, 216-217), trim_limits against a
brute-force statement of tests/test_packed_attention.py:53-57, and the JAX module's import
behaviour where jax is absent."""
import importlib.util

import numpy as np
import pytest
import torch

from colabfold_legacy_kernels import layouts, torch_ops


def test_transposes():
    rng = np.random.default_rng(0)
    wp, wg = rng.standard_normal((64, 256)), rng.standard_normal((64, 256))
    wpT, wgT = layouts.proj_pair_T(wp, wg)
    assert wpT.shape == (256, 64) and wpT.flags.c_contiguous
    for p, k in ((0, 0), (255, 63), (17, 40)):
        assert wpT[p, k] == wp[k, p] and wgT[p, k] == wg[k, p]
    w = torch.from_numpy(rng.standard_normal((128, 64)))
    wT = layouts.linear_T(w)
    assert wT.shape == (64, 128) and wT.is_contiguous() and wT[5, 100] == w[100, 5]
    wb = rng.standard_normal((128, 4))
    assert layouts.heads_T(wb)[3, 77] == wb[77, 3]


@pytest.mark.parametrize("lib", ("numpy", "torch"))
def test_slot_major(lib):
    rng = np.random.default_rng(1)
    w = rng.standard_normal((4, 64, 128))
    if lib == "torch":
        w = torch.from_numpy(w)
    wT = layouts.slot_major(w)
    assert tuple(wT.shape) == (512, 64)
    for s, k, j in ((0, 0, 0), (3, 63, 127), (2, 10, 99), (1, 33, 0)):
        assert wT[s * 128 + j, k] == w[s, k, j]


@pytest.mark.parametrize("lib", ("numpy", "torch"))
def test_w2_blocked(lib):
    rng = np.random.default_rng(2)
    w2 = rng.standard_normal((256, 64))
    if lib == "torch":
        w2 = torch.from_numpy(w2)
    w2T = layouts.w2_blocked(w2)
    assert tuple(w2T.shape) == (4, 64, 64)
    for j, c, i in ((0, 0, 0), (3, 63, 63), (1, 17, 5), (2, 40, 33)):
        assert w2T[j, c, i] == w2[64 * j + i, c]
    back = layouts.w2_unblocked(w2T)
    assert (np.asarray(back) == np.asarray(w2)).all()
    with pytest.raises(ValueError):
        layouts.w2_blocked(w2[:100])


def brute_lims(km):
    n, s = km.shape
    last = []
    for r in range(n):
        live = [j for j in range(s) if km[r, j]]
        last.append(live[-1] + 1 if live else 0)
    return last + [max(last) if last else 0]


@pytest.mark.parametrize("shape", [(5, 9), (1, 1), (4, 0), (0, 7), (64, 300)])
def test_trim_limits(shape):
    rng = np.random.default_rng(3)
    km = (rng.random(shape) > 0.6).astype(np.uint8)
    if shape[0] > 2 and shape[1] > 0:
        km[1] = 0          # a row with no live key
        km[2, -1] = 1      # a row live up to the end
    got = torch_ops.trim_limits(torch.from_numpy(km))
    assert got.dtype == torch.int32 and got.tolist() == brute_lims(km)


def test_fused_available_declines():
    """Other widths and dtypes decline (tests/test_fused.py:223-229)."""
    f16 = torch.float16
    assert torch_ops.fused_available("ln_gated_dual_proj", f16, 128, 128)
    assert not torch_ops.fused_available("ln_gated_dual_proj", f16, 256, 128)
    assert not torch_ops.fused_available("ln_projection", f16, 128, 32)
    assert not torch_ops.fused_available("output_projection", f16, 256, 256)
    assert not torch_ops.fused_available("ln_projection", f16, 256, 256)
    assert torch_ops.fused_available("ln_projection", torch.bfloat16, 128, 128)  # an addition here
    assert not torch_ops.fused_available("ln_projection", torch.float32, 128, 128)
    assert not torch_ops.fused_available("transition", f16, 512, 2048)
    assert not torch_ops.fused_available("transition", f16, 128, 384)
    assert torch_ops.fused_available("transition", f16, 256, 1024)


def test_jax_module_without_jax():
    from colabfold_legacy_kernels import jax_ops
    assert len(set(jax_ops.HANDLERS)) == 13
    assert {"VoltaMma", "VoltaMmaBwd", "VoltaMmaPacked", "VoltaMmaPackedTrim", "VoltaOpmOuter"} <= set(
        jax_ops.HANDLERS)
    if importlib.util.find_spec("jax") is None:
        with pytest.raises(ImportError):
            jax_ops.register()
