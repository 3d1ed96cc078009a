"""PyTorch-ROCm front end of the gfx950 library: each function is one XLA FFI target of the
reference, called through the library's C ABI (include/colabfold_gfx950.h) on the current HIP
stream, with the FFI binding's buffer order, attributes, result shapes and error behaviour.

  attention_fwd       VoltaMma            (reference cuda/volta_mma_attn.cu:625-640)
  attention_packed    VoltaMmaPacked[Trim] (volta_mma_attn.cu:594-623)
  attention_bwd       VoltaMmaBwd         (cuda/volta_mma_attn_bwd.cu:455-473)
  ln_gdp              VoltaLnGdp          (cuda/volta_fused_ffi.h:337-351)
  trimul_epilogue     VoltaTrimulEpilogue (volta_fused_ffi.h:353-371)
  ln_projection       VoltaLnProj         (volta_fused_ffi.h:373-388)
  output_projection   VoltaOutProj        (volta_fused_ffi.h:390-401)
  transition          VoltaTransition     (volta_fused_ffi.h:403-418)
  layer_norm          VoltaLayerNorm      (cuda/volta_ops.cu:86-94)
  gated_dual_proj     VoltaGdp            (volta_ops.cu:258-269)

Results are allocated here with torch (as XLA preallocates them) unless passed in, which is how a
caller aliases an output to its residual / input. The fused ops take fp16 or bf16 activations
(all of a call's activations and results one type; weights, biases and keep fp16); results come
back in the activation type. A rejected call raises InvalidArgument (the
FFI's InvalidArgument) and a launch failure KernelError (Internal), with the library's message.
There is no CPU fallback: without the built library every call raises.
"""
import ctypes

import torch

from . import library_path

CLK_S32, CLK_U8, CLK_F16, CLK_F32, CLK_BF16 = 4, 6, 10, 11, 16
_DTYPES = {torch.int32: CLK_S32, torch.uint8: CLK_U8, torch.float16: CLK_F16,
           torch.float32: CLK_F32, torch.bfloat16: CLK_BF16}
INVALID_ARGUMENT, INTERNAL = 3, 13


class KernelError(RuntimeError):
    def __init__(self, code, message):
        super().__init__(message)
        self.code = code


class InvalidArgument(KernelError, ValueError):
    pass


class Buffer(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("dtype", ctypes.c_int32), ("rank", ctypes.c_int32),
                ("dims", ctypes.POINTER(ctypes.c_int64))]


_P = ctypes.POINTER(Buffer)
_lib = None

_SIGNATURES = {
    "clk_attention_fwd": [ctypes.c_void_p, ctypes.c_int32] + [_P] * 7 +
                         [ctypes.c_float, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32],
    "clk_attention_packed": [ctypes.c_void_p, ctypes.c_int32] + [_P] * 5 +
                            [ctypes.c_float, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32],
    "clk_attention_packed_trim": [ctypes.c_void_p, ctypes.c_int32] + [_P] * 6 +
                                 [ctypes.c_float, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32],
    "clk_attention_bwd": [ctypes.c_void_p, ctypes.c_int32] + [_P] * 12 +
                         [ctypes.c_float, ctypes.c_int32, ctypes.c_void_p, ctypes.c_size_t],
    "clk_attention_bwd_noalloc": [ctypes.c_void_p, ctypes.c_int32] + [_P] * 12 +
                                 [ctypes.c_float, ctypes.c_int32],
    "clk_ln_gdp": [ctypes.c_void_p] + [_P] * 10 + [ctypes.c_float],
    "clk_trimul_epilogue": [ctypes.c_void_p] + [_P] * 12 +
                           [ctypes.c_float, ctypes.c_int32, ctypes.c_int32],
    "clk_ln_projection": [ctypes.c_void_p] + [_P] * 8 +
                         [ctypes.c_float, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32],
    "clk_output_projection": [ctypes.c_void_p] + [_P] * 6 + [ctypes.c_int32, ctypes.c_int32],
    "clk_transition": [ctypes.c_void_p] + [_P] * 9 +
                      [ctypes.c_float, ctypes.c_int32, ctypes.c_int32],
    "clk_layer_norm": [ctypes.c_void_p] + [_P] * 4 + [ctypes.c_float],
    "clk_gated_dual_proj": [ctypes.c_void_p, ctypes.c_int32] + [_P] * 7 + [ctypes.c_int64],
    "clk_opm_update": [ctypes.c_void_p] + [_P] * 6 + [ctypes.c_float, ctypes.c_int32],
    "clk_opm_outer": [ctypes.c_void_p] + [_P] * 4,
}


def lib():
    """The loaded gfx950 library (raises FileNotFoundError when it is not built)."""
    global _lib
    if _lib is None:
        handle = ctypes.CDLL(library_path("attention", 950))
        for name, args in _SIGNATURES.items():
            fn = getattr(handle, name)  # a library missing an entry point fails here, loudly
            fn.argtypes = args
            fn.restype = ctypes.c_int
        handle.clk_last_error.restype = ctypes.c_char_p
        handle.clk_version.restype = ctypes.c_char_p
        handle.clk_attention_bwd_workspace_size.argtypes = [ctypes.c_int32, _P, _P]
        handle.clk_attention_bwd_workspace_size.restype = ctypes.c_size_t
        handle.clk_attention_bwd_plan.argtypes = [ctypes.c_int32] + [ctypes.c_int64] * 5 + \
            [ctypes.POINTER(ctypes.c_int64), ctypes.c_int32]
        handle.clk_attention_bwd_plan.restype = ctypes.c_int
        handle.clk_attention_bwd_noalloc_scratch_size.argtypes = []
        handle.clk_attention_bwd_noalloc_scratch_size.restype = ctypes.c_size_t
        _lib = handle
    return _lib


def buffer(t):
    """A clk_buffer describing tensor t (contiguous, on a HIP device)."""
    if t.dtype not in _DTYPES:
        raise TypeError("unsupported dtype %s" % t.dtype)
    if not t.is_contiguous():
        raise ValueError("tensors must be contiguous")
    dims = (ctypes.c_int64 * max(t.dim(), 1))(*t.shape)
    b = Buffer(ctypes.c_void_p(t.data_ptr()), _DTYPES[t.dtype], t.dim(), dims)
    b._keep = dims
    return b


def _ref(b):
    return ctypes.byref(b)


def _check(status):
    if status != 0:
        msg = lib().clk_last_error().decode()
        if status == INVALID_ARGUMENT:
            raise InvalidArgument(status, msg)
        raise KernelError(status, msg)


def _stream(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


_ONES = {}


def _one(like, dtype):
    """The one-element buffer the FFI takes for an absent optional input, or for a result that is
    not produced (never written, never returned). One zero buffer per device and dtype is kept for
    the process, so a call adds no allocation or fill of its own."""
    key = (like.device, dtype)
    t = _ONES.get(key)
    if t is None:
        t = _ONES[key] = torch.zeros(1, dtype=dtype, device=like.device)
    return t


def attention_fwd(q, k, v, bias, kmask, scale, block_q=64, block_k=32, want_lse=True, out=None,
                  lse=None):
    """VoltaMma: out [N,H,Sq,D] F16 and lse [N,H,Sq] F32 (log2 domain), or a one-element lse
    left untouched without want_lse (tests/test_attn_bwd.py:47-57)."""
    n, h, sq, d = q.shape
    out = torch.empty_like(q) if out is None else out
    if lse is None:
        lse = (torch.empty((n, h, sq), dtype=torch.float32, device=q.device) if want_lse
               else torch.zeros(1, dtype=torch.float32, device=q.device))
    bufs = [buffer(t) for t in (q, k, v, bias, kmask, out, lse)]
    _check(lib().clk_attention_fwd(_stream(q), q.device.index, *map(_ref, bufs), float(scale),
                                   int(block_q), int(block_k), int(bool(want_lse))))
    return out, lse


def attention_packed(p, bias, kmask, gate_bias, scale, block_q=64, block_k=32, column=False,
                     lims=None, out=None):
    """VoltaMmaPacked (lims None) or VoltaMmaPackedTrim: out [X,Y,H,D] F16 from p [X,Y,G,H,D]."""
    x, y, _, h, d = p.shape
    out = torch.empty((x, y, h, d), dtype=torch.float16, device=p.device) if out is None else out
    if lims is None:
        bufs = [buffer(t) for t in (p, bias, kmask, gate_bias, out)]
        fn = lib().clk_attention_packed
    else:
        bufs = [buffer(t) for t in (p, bias, kmask, gate_bias, lims, out)]
        fn = lib().clk_attention_packed_trim
    _check(fn(_stream(p), p.device.index, *map(_ref, bufs), float(scale), int(block_q),
              int(block_k), int(bool(column))))
    return out


def attention_bwd_workspace(q, k):
    return int(lib().clk_attention_bwd_workspace_size(q.device.index, _ref(buffer(q)),
                                                      _ref(buffer(k))))


def attention_bwd_plan(n, h, sq, sk, d, device=0):
    """The backward's launch plan on `device` (a diagnostic for tests and the bench)."""
    vals = (ctypes.c_int64 * 6)()
    _check(lib().clk_attention_bwd_plan(device, n, h, sq, sk, d, vals, 6))
    return dict(zip(("row_groups", "chunk", "chunks", "passes", "windows", "registers"), list(vals)))


def attention_bwd(q, k, v, bias, kmask, out, dout, lse, scale, want_dbias=True, workspace=None,
                  grads=None):
    """VoltaMmaBwd: dq, dk, dv F16 and dbias [H,Sq,Sk] F32 (zeros without want_dbias), written
    into `grads` = (dq, dk, dv, dbias) when given, as into XLA's preallocated results."""
    if grads is None:
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        dbias = torch.empty(bias.shape, dtype=torch.float32, device=q.device)
    else:
        dq, dk, dv, dbias = grads
    if workspace is None:
        need = attention_bwd_workspace(q, k)
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    bufs = [buffer(t) for t in (q, k, v, bias, kmask, out, dout, lse, dq, dk, dv, dbias)]
    _check(lib().clk_attention_bwd(_stream(q), q.device.index, *map(_ref, bufs), float(scale),
                                   int(bool(want_dbias)), ctypes.c_void_p(workspace.data_ptr()),
                                   workspace.numel()))
    return dq, dk, dv, dbias


def attention_bwd_noalloc(q, k, v, bias, kmask, out, dout, lse, scale, want_dbias=True,
                          grads=None):
    """VoltaMmaBwd without a workspace: the library's static per-GPU scratch serves instead
    (clk_attention_bwd_noalloc; calls that overlap on one GPU race for it)."""
    if grads is None:
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        dbias = torch.empty(bias.shape, dtype=torch.float32, device=q.device)
    else:
        dq, dk, dv, dbias = grads
    bufs = [buffer(t) for t in (q, k, v, bias, kmask, out, dout, lse, dq, dk, dv, dbias)]
    _check(lib().clk_attention_bwd_noalloc(_stream(q), q.device.index, *map(_ref, bufs),
                                           float(scale), int(bool(want_dbias))))
    return dq, dk, dv, dbias


def ln_gdp(x, scale, offset, wpT, bp, wgT, bg, mask, eps=1e-5):
    """VoltaLnGdp: left, right [P/2, M] F16, channel major."""
    m, p = x.shape[0], wpT.shape[0]
    left = torch.empty((p // 2, m), dtype=x.dtype, device=x.device)
    right = torch.empty((p // 2, m), dtype=x.dtype, device=x.device)
    bufs = [buffer(t) for t in (x, scale, offset, wpT, bp, wgT, bg, mask, left, right)]
    _check(lib().clk_ln_gdp(_stream(x), *map(_ref, bufs), float(eps)))
    return left, right


def trimul_epilogue(x_cm, x, in_scale, in_offset, ln_scale, ln_offset, woT, bo, wgT, bg,
                    keep=None, eps=1e-5, add_input=False, out=None):
    """VoltaTrimulEpilogue: out [M,O] F16. out may be x itself with add_input."""
    m, o = x.shape[0], woT.shape[0]
    out = torch.empty((m, o), dtype=x.dtype, device=x.device) if out is None else out
    has_keep = keep is not None
    keep = keep if has_keep else _one(x, torch.float16)
    bufs = [buffer(t) for t in (x_cm, x, in_scale, in_offset, ln_scale, ln_offset, woT, bo, wgT,
                                bg, keep, out)]
    _check(lib().clk_trimul_epilogue(_stream(x), *map(_ref, bufs), float(eps),
                                     int(bool(add_input)), int(has_keep)))
    return out


def ln_projection(x, scale, offset, wT=None, wbT=None, keep=None, eps=1e-5):
    """VoltaLnProj: p [M,n] = LN(x)@w and bias [heads,M]; a missing weight gives n or heads 0
    and a one-element (untouched) result in its place."""
    m = x.shape[0]
    n = 0 if wT is None else wT.shape[0]
    heads = 0 if wbT is None else wbT.shape[0]
    p = torch.empty((m, n), dtype=x.dtype, device=x.device) if n else _one(x, x.dtype)
    bias = (torch.empty((heads, m), dtype=x.dtype, device=x.device) if heads
            else _one(x, x.dtype))
    has_keep = keep is not None
    keep = keep if has_keep else _one(x, torch.float16)
    wT = wT if n else _one(x, torch.float16)
    wbT = wbT if heads else _one(x, torch.float16)
    bufs = [buffer(t) for t in (x, scale, offset, wT, wbT, keep, p, bias)]
    _check(lib().clk_ln_projection(_stream(x), *map(_ref, bufs), float(eps), n, heads,
                                   int(has_keep)))
    return (p if n else None), (bias if heads else None)


def output_projection(o, wT, b, residual=None, keep=None, out=None):
    """VoltaOutProj: out [M,N] = o@w + b [+ residual]; out may be residual itself."""
    m, n = o.shape[0], wT.shape[0]
    out = torch.empty((m, n), dtype=o.dtype, device=o.device) if out is None else out
    has_residual = residual is not None
    residual = residual if has_residual else _one(o, o.dtype)
    has_keep = keep is not None
    keep = keep if has_keep else _one(o, torch.float16)
    bufs = [buffer(t) for t in (o, wT, b, residual, keep, out)]
    _check(lib().clk_output_projection(_stream(o), *map(_ref, bufs), int(has_residual),
                                       int(has_keep)))
    return out


def transition(x, scale, offset, w1T, b1, w2T, b2, keep=None, eps=1e-5, add_input=False,
               out=None):
    """VoltaTransition: out [M,C] = relu(LN(x)@w1 + b1)@w2 + b2 [+ x], w2T blocked
    [H/64][C][64]; out may be x itself with add_input."""
    out = torch.empty_like(x) if out is None else out
    has_keep = keep is not None
    keep = keep if has_keep else _one(x, torch.float16)
    bufs = [buffer(t) for t in (x, scale, offset, w1T, b1, w2T, b2, keep, out)]
    _check(lib().clk_transition(_stream(x), *map(_ref, bufs), float(eps), int(bool(add_input)),
                                int(has_keep)))
    return out


def layer_norm(x, scale, offset, eps=1e-5, out=None):
    """VoltaLayerNorm: out [M,C] F16, one-pass fp32 statistics."""
    out = torch.empty_like(x) if out is None else out
    bufs = [buffer(t) for t in (x, scale, offset, out)]
    _check(lib().clk_layer_norm(_stream(x), *map(_ref, bufs), float(eps)))
    return out


def gated_dual_proj(x, wp, bp, wg, bg, mask, activation=0, out=None):
    """VoltaGdp: out [M,N] = mask * (x@wp + bp) * act(x@wg + bg); wp, wg [K,N];
    activation 0 sigmoid, 1 swish."""
    m, n = x.shape[0], wp.shape[1]
    out = torch.empty((m, n), dtype=torch.float16, device=x.device) if out is None else out
    bufs = [buffer(t) for t in (x, wp, bp, wg, bg, mask, out)]
    _check(lib().clk_gated_dual_proj(_stream(x), x.device.index, *map(_ref, bufs), int(activation)))
    return out


def opm_update(lhs, t, bias, norm, residual=None, eps=1e-3, out=None):
    """VoltaOpmUpdate: out [B,D,F] = (lhs@t[:, d] + bias) / (eps + norm[b, d]) (+ residual);
    lhs [B,K], t [K,D,F] fp16, bias [F], norm [B,D] fp32. residual may be `out` itself."""
    b, (d, f) = lhs.shape[0], t.shape[1:]
    out = torch.empty((b, d, f), dtype=torch.float16, device=lhs.device) if out is None else out
    res = residual if residual is not None else _one(lhs, torch.float16)
    bufs = [buffer(x) for x in (lhs, t, bias, norm, res, out)]
    _check(lib().clk_opm_update(_stream(lhs), *map(_ref, bufs), float(eps), int(residual is not None)))
    return out


def opm_outer(left, right, wT, out=None):
    """VoltaOpmOuter: out [B,D,F] = sum_c,e f16(sum_a left[a,b,c] right[a,d,e]) wT[f, c*32 + e];
    left [16,B,C], right [16,D,32], wT [F, 32 C], all fp16."""
    b, d, f = left.shape[1], right.shape[1], wT.shape[0]
    out = torch.empty((b, d, f), dtype=torch.float16, device=left.device) if out is None else out
    bufs = [buffer(x) for x in (left, right, wT, out)]
    _check(lib().clk_opm_outer(_stream(left), *map(_ref, bufs)))
    return out
