"""Caller glue for PyTorch: what the reference's callers wrap around the FFI targets.

The reference repository ships the FFI targets only; its callers (the external
colabfold_kernels package) wire them into the framework. Its tests show the pieces this module
provides on top of `hip` (the C ABI binding):

  attention        the forward + backward pair as one differentiable op: VoltaMma with want_lse,
                   its lse kept for VoltaMmaBwd, and dbias cast to the bias dtype
                   (tests/test_attn_bwd.py:262-281, the custom_vjp wiring)
  gated_attention  attention times sigmoid(gate + gate_bias), the gated packed forward's
                   epilogue (cuda/volta_attn.h:46-52) as a differentiable op, so the gate gets
                   its gradient
  trim_limits      each batch row's last live key + 1, then the largest: the lims of
                   VoltaMmaPackedTrim (tests/test_packed_attention.py:53-57)
  ln_gated_dual_proj, trimul_epilogue_ln, ln_projection, output_projection, transition
                   the fused targets with the callers' natural weight shapes, re-laid out by
                   colabfold_legacy_kernels.layouts, and leading batch dimensions folded into
                   the row count (tests/test_fused.py:96-229 calls them so)
  fused_available  whether a fused target takes a width and dtype (tests/test_fused.py:223-229:
                   other widths and dtypes decline to the caller's own path)

Everything runs on the GPU through the built library; there is no CPU path. The fused wrappers
are forward only (the reference's callers take their gradients from jnp references). They take
fp16 or bf16 activations, with weights and biases cast to fp16 for the kernels.
"""
import torch

from . import hip
from . import layouts

# (D, block_q, block_k) each head dim runs with by default: an entry of the reference's forward
# dispatch set (cuda/volta_mma_attn.cu:508-517), (64, 64) where D = 64 has no (64, 32)
_DEFAULT_BLOCKS = {8: (64, 32), 16: (64, 32), 24: (64, 32), 32: (64, 32), 48: (64, 32),
                   64: (64, 64), 96: (64, 32)}


def default_blocks(d):
    if d not in _DEFAULT_BLOCKS:
        raise hip.InvalidArgument(hip.INVALID_ARGUMENT, "attention: unsupported head dim %d" % d)
    return _DEFAULT_BLOCKS[d]


class _Attention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, bias, kmask, scale, block_q, block_k):
        q, k, v, bias, kmask = (t.contiguous() for t in (q, k, v, bias, kmask))
        out, lse = hip.attention_fwd(q, k, v, bias, kmask, scale, block_q, block_k, want_lse=True)
        ctx.save_for_backward(q, k, v, bias, kmask, out, lse)
        ctx.scale = scale
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, bias, kmask, out, lse = ctx.saved_tensors
        want_dbias = bool(ctx.needs_input_grad[3])
        dq, dk, dv, dbias = hip.attention_bwd(q, k, v, bias, kmask, out,
                                              dout.to(torch.float16).contiguous(), lse, ctx.scale,
                                              want_dbias=want_dbias)
        return dq, dk, dv, (dbias.to(bias.dtype) if want_dbias else None), None, None, None, None


def attention(q, k, v, bias, kmask, scale=None, block_q=None, block_k=None):
    """Biased, masked attention [N,H,Sq,D] fp16, differentiable in q, k, v and bias.

    q [N,H,Sq,D], k, v [N,H,Sk,D], bias [H,Sq,Sk] fp16; kmask [N,Sk] (nonzero keeps a key).
    scale defaults to D^-1/2. The backward is VoltaMmaBwd with want_dbias only where bias needs
    a gradient; dbias (fp32, summed over the N rows) is cast to the bias dtype.
    """
    d = q.shape[-1]
    bq, bk = default_blocks(d) if block_q is None else (block_q, block_k)
    if kmask.dtype != torch.uint8:
        kmask = (kmask != 0).to(torch.uint8)
    return _Attention.apply(q, k, v, bias, kmask, float(d ** -0.5 if scale is None else scale),
                            int(bq), int(bk))


def gated_attention(q, k, v, bias, kmask, gate, gate_bias=None, scale=None):
    """attention(...) * sigmoid(gate + gate_bias), differentiable in the gate too.

    gate [N,H,Sq,D]; gate_bias [H,D] or [H*D] (zeros if None). The attention output o comes back
    from the kernel already rounded to fp16; the product o * sigmoid(g) is taken in fp32 and
    rounded to fp16 again. The result therefore carries two roundings, where the reference's gated
    packed forward gates the fp32 output and rounds once (cuda/volta_attn.h:46-52): the two
    differ by at most about one fp16 ulp of the result (|sigmoid| <= 1, so o's rounding error of
    half an ulp of o is at most half an ulp of the product's scale, plus the product's own half
    ulp). VoltaMmaPacked with G = 4 (attention_packed) is the single-rounding forward."""
    o = attention(q, k, v, bias, kmask, scale)
    g = gate.float()
    if gate_bias is not None:
        h, d = q.shape[1], q.shape[3]
        g = g + gate_bias.float().reshape(1, h, 1, d)
    return (o.float() * torch.sigmoid(g)).to(torch.float16)


def trim_limits(kmask):
    """lims [N+1] int32 on kmask's device: for each batch row its last live key + 1 (0 when the
    row has none), then the largest of them (tests/test_packed_attention.py:53-57)."""
    live = kmask != 0
    n, s = live.shape
    pos = torch.arange(1, s + 1, device=kmask.device, dtype=torch.int32)
    last = torch.where(live, pos, torch.zeros((), dtype=torch.int32, device=kmask.device))
    last = last.amax(dim=1) if s > 0 else torch.zeros(n, dtype=torch.int32, device=kmask.device)
    top = last.amax().reshape(1) if n > 0 else torch.zeros(1, dtype=torch.int32, device=kmask.device)
    return torch.cat([last, top]).to(torch.int32).contiguous()


# ---- fused pair-stack ops with natural weight shapes ----------------------------------------

def fused_available(kernel, dtype, *widths):
    """True if `kernel` takes these widths and this activation dtype: ln_gated_dual_proj (a, ci),
    trimul_epilogue (a, ci), ln_projection (a, n), output_projection (k, c), transition (c,
    hidden). fp16 is the reference's F16 contract; bf16 activations are this library's addition
    (the reference's wrappers decline them, tests/test_fused.py:223-229)."""
    if dtype not in (torch.float16, torch.bfloat16):
        return False
    w2 = {64, 128}
    if kernel in ("ln_gated_dual_proj", "trimul_epilogue"):
        a, ci = widths
        return a in w2 and ci in w2
    if kernel == "ln_projection":
        a = widths[0]
        n = widths[1] if len(widths) > 1 else 0
        return a in w2 and (n == 0 or n % 64 == 0)
    if kernel == "output_projection":
        k, c = widths
        return k in w2 and c in w2
    if kernel == "transition":
        c, hd = widths
        return c in (64, 128, 256) and hd in (2 * c, 4 * c)
    raise KeyError(kernel)


def _rows(x):
    """x [..., C] -> ([M, C] contiguous, leading shape)."""
    return x.reshape(-1, x.shape[-1]).contiguous(), tuple(x.shape[:-1])


def _keep_rows(keep):
    return None if keep is None else keep.reshape(-1).to(torch.float16).contiguous()


def _w16(w):
    """Weights and biases go to the kernels as fp16."""
    return w.to(torch.float16)


def ln_gated_dual_proj(x, scale, offset, wp, bp, wg, bg, mask, eps=1e-5):
    """left, right [ci, M] (channel major) = the halves of mask (LN(x)@wp + bp) sigmoid(LN(x)@wg
    + bg), with wp, wg [a, 2 ci] (tests/test_fused.py:96-103)."""
    x2, _ = _rows(x)
    wpT, wgT = layouts.proj_pair_T(_w16(wp), _w16(wg))
    return hip.ln_gdp(x2, scale.float().contiguous(), offset.float().contiguous(), wpT,
                      _w16(bp).contiguous(), wgT, _w16(bg).contiguous(), _keep_rows(mask), eps)


def trimul_epilogue_ln(x_cm, x, in_scale, in_offset, ln_scale, ln_offset, wo, bo, wg, bg,
                       keep=None, add_input=False, eps=1e-5):
    """out [..., a] = (LN(x_cm^T)@wo + bo) sigmoid(LN_in(x)@wg + bg) (+ x), with x_cm [ci, M]
    fp32, wo [ci, a], wg [a, a] (tests/test_fused.py:104-121). With add_input the result is
    written over x, as the target's output aliases its input."""
    x2, lead = _rows(x)
    out = hip.trimul_epilogue(x_cm.float().contiguous(), x2, in_scale.float().contiguous(),
                              in_offset.float().contiguous(), ln_scale.float().contiguous(),
                              ln_offset.float().contiguous(), layouts.linear_T(_w16(wo)),
                              _w16(bo).contiguous(), layouts.linear_T(_w16(wg)),
                              _w16(bg).contiguous(), keep=_keep_rows(keep), eps=eps,
                              add_input=add_input, out=x2 if add_input else None)
    return out.reshape(lead + (out.shape[-1],))


def ln_projection(x, scale, offset, w=None, wb=None, keep=None, eps=1e-5):
    """p [..., slots, n] = LN(x)@w[s] for each slot (no bias term) and the head bias
    [heads, ...] = (LN(x)@wb)^T, with w [slots, a, n] and wb [a, heads]; either may be None
    (tests/test_fused.py:180-199)."""
    x2, lead = _rows(x)
    wT = None if w is None else layouts.slot_major(_w16(w))
    wbT = None if wb is None else layouts.heads_T(_w16(wb))
    p, b = hip.ln_projection(x2, scale.float().contiguous(), offset.float().contiguous(), wT, wbT,
                             keep=_keep_rows(keep), eps=eps)
    if p is not None:
        p = p.reshape(lead + (w.shape[0], w.shape[2]))
    if b is not None:
        b = b.reshape((b.shape[0],) + lead)
    return p, b


def output_projection(o, w, b, residual=None, keep=None):
    """out [..., c] = o@w + b (+ residual), w [k, c]; with a residual the result is written over
    it, as the target aliases them (tests/test_fused.py:201-213)."""
    o2, lead = _rows(o)
    r2 = None if residual is None else residual.reshape(-1, residual.shape[-1]).contiguous()
    out = hip.output_projection(o2, layouts.linear_T(_w16(w)), _w16(b).contiguous(), residual=r2,
                                keep=_keep_rows(keep), out=r2)
    return out.reshape(lead + (out.shape[-1],))


def transition(x, scale, offset, w1, b1, w2, b2, keep=None, add_input=False, eps=1e-5):
    """out [..., c] = relu(LN(x)@w1 + b1)@w2 + b2 (+ x), w1 [c, hidden], w2 [hidden, c]
    (tests/test_fused.py:215-229); with add_input the result is written over x."""
    x2, lead = _rows(x)
    out = hip.transition(x2, scale.float().contiguous(), offset.float().contiguous(),
                         layouts.linear_T(_w16(w1)), _w16(b1).contiguous(),
                         layouts.w2_blocked(_w16(w2)), _w16(b2).contiguous(),
                         keep=_keep_rows(keep), eps=eps, add_input=add_input,
                         out=x2 if add_input else None)
    return out.reshape(lead + (out.shape[-1],))
