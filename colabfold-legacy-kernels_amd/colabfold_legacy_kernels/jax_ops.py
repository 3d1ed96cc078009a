"""Caller glue for JAX (jaxlib with ROCm): registration of the gfx950 handler symbols as XLA FFI
targets, and attention as a custom_vjp over VoltaMma / VoltaMmaBwd.

jax is imported on first use only, so this module imports everywhere; calling into it without
jax raises ImportError. It follows the reference's own wiring: registration and the two
ffi_call forms of tests/test_attn_bwd.py:37-71 (platform "ROCM" instead of "CUDA"), and the
custom_vjp of tests/test_attn_bwd.py:262-281 (the forward's lse kept for the backward, dbias
cast to the bias dtype). The fused targets are called with the layouts of
colabfold_legacy_kernels.layouts, as in the PyTorch glue (torch_ops).

jax is not installed where this repository is tested, so this module is not exercised by its
tests beyond importing; the PyTorch glue (torch_ops) carries the same logic and is tested.
"""
import ctypes

import numpy as np

from . import KERNELS, library_path, symbol

# every handler symbol the library exports: the locator's eleven kernels, plus the packed
# forwards that sit beside VoltaMma in the reference's attention library
HANDLERS = tuple(symbol(k, 950) for k in KERNELS) + ("VoltaMmaPacked", "VoltaMmaPackedTrim")

_registered = set()


def _jax():
    try:
        import jax
        import jax.numpy as jnp
    except ImportError as e:  # pragma: no cover - depends on the environment
        raise ImportError("colabfold_legacy_kernels.jax_ops needs jax with a ROCm jaxlib") from e
    return jax, jnp


def register(platform="ROCM"):
    """Register every handler symbol of the gfx950 library as an XLA FFI target (once)."""
    jax, _ = _jax()
    if platform in _registered:
        return
    lib = ctypes.cdll.LoadLibrary(str(library_path("attention", 950)))
    for name in HANDLERS:
        jax.ffi.register_ffi_target(name, jax.ffi.pycapsule(getattr(lib, name)), platform=platform)
    _registered.add(platform)


def attention_fwd(q, k, v, bias, kmask, scale, block_q=64, block_k=32, want_lse=True):
    """VoltaMma: (out [N,H,Sq,D] f16, lse [N,H,Sq] f32), or a one-element lse without want_lse."""
    jax, jnp = _jax()
    n, h, sq, d = q.shape
    lse_shape = (n, h, sq) if want_lse else (1,)
    return jax.ffi.ffi_call(
        "VoltaMma",
        (jax.ShapeDtypeStruct((n, h, sq, d), jnp.float16),
         jax.ShapeDtypeStruct(lse_shape, jnp.float32)),
        vmap_method="sequential")(
            q, k, v, bias, kmask, scale=np.float32(scale), block_q=np.int64(block_q),
            block_k=np.int64(block_k), want_lse=bool(want_lse))


def attention_bwd(q, k, v, bias, kmask, out, dout, lse, scale, want_dbias=True):
    """VoltaMmaBwd: (dq, dk, dv f16, dbias [H,Sq,Sk] f32)."""
    jax, jnp = _jax()
    h, sq, sk = q.shape[1], q.shape[2], k.shape[2]
    return jax.ffi.ffi_call(
        "VoltaMmaBwd",
        (jax.ShapeDtypeStruct(q.shape, jnp.float16), jax.ShapeDtypeStruct(k.shape, jnp.float16),
         jax.ShapeDtypeStruct(v.shape, jnp.float16), jax.ShapeDtypeStruct((h, sq, sk), jnp.float32)),
        vmap_method="sequential")(
            q, k, v, bias, kmask, out, dout, lse, scale=np.float32(scale),
            want_dbias=bool(want_dbias))


def make_attention(kmask, scale, block_q=64, block_k=32):
    """attention(q, k, v, bias) with this key mask and scale, differentiable in all four
    (the custom_vjp of tests/test_attn_bwd.py:262-281)."""
    jax, _ = _jax()
    register()

    @jax.custom_vjp
    def attention(q, k, v, bias):
        return attention_fwd(q, k, v, bias, kmask, scale, block_q, block_k)[0]

    def fwd(q, k, v, bias):
        out, lse = attention_fwd(q, k, v, bias, kmask, scale, block_q, block_k)
        return out, (q, k, v, bias, out, lse)

    def bwd(res, dout):
        q, k, v, bias, out, lse = res
        dq, dk, dv, dbias = attention_bwd(q, k, v, bias, kmask, out, dout, lse, scale)
        return dq, dk, dv, dbias.astype(bias.dtype)

    attention.defvjp(fwd, bwd)
    return attention
