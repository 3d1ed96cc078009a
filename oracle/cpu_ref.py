"""torch-CPU float32 restatement of the reference tests' plain jnp ops (TEST INFRASTRUCTURE ONLY).

The reference checks its kernels against jnp on XLA: attention as the four-line reference() of
tests/test_attn_bwd.py:74-79 (fp32 einsum, bias, the replace mask -1e4, softmax, einsum), its
gradients by jax.grad, and the fused ops against colabfold-kernels' fp32 closed forms. jax is not
installed here or on the GPU box, so this module states the same fp32 math in torch on the CPU;
bench.py times it as the CPU baseline ("port", a baseline and not the target) on a bounded
sample of the benchmark workload. It is not a checker: the float64 oracle (attention.py,
fused.py) is.
"""
import torch

MASKED_LOGIT = -1.0e4


def attention(q, k, v, bias, kmask, scale):
    """fp32 attention with the kernels' masking convention (tests/test_attn_bwd.py:74-79)."""
    logits = scale * torch.einsum("nhqd,nhkd->nhqk", q, k) + bias[None]
    logits = torch.where(kmask[:, None, None, :] != 0, logits, torch.tensor(MASKED_LOGIT))
    p = torch.softmax(logits, dim=-1)
    return torch.einsum("nhqk,nhkd->nhqd", p, v)


def attention_fwd_bwd(q, k, v, bias, kmask, dout, scale):
    """out and dq, dk, dv, dbias by autograd, in fp32 on the CPU."""
    q, k, v, bias = (t.detach().float().requires_grad_(True) for t in (q, k, v, bias))
    out = attention(q, k, v, bias, kmask, scale)
    out.backward(dout.float())
    return out.detach(), q.grad, k.grad, v.grad, bias.grad


def layer_norm(x, scale, offset, eps):
    return torch.nn.functional.layer_norm(x.float(), (x.shape[-1],), scale, offset, eps)


def ln_projection(x, scale, offset, wT, wbT, eps):
    y = layer_norm(x, scale, offset, eps)
    return y @ wT.float().T, (y @ wbT.float().T).T


def transition(x, scale, offset, w1T, b1, w2, b2, eps):
    y = layer_norm(x, scale, offset, eps)
    return torch.relu(y @ w1T.float().T + b1.float()) @ w2.float() + b2.float() + x.float()
