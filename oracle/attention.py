"""Float64 oracle for biased, masked, optionally gated flash attention (TEST INFRASTRUCTURE ONLY).

Restates the math of the reference attention kernels, not their tiling:
  forward   cuda/volta_mma_attn.cu:317-464 (scale, bias, mask, softmax, lse, gate),
            closed form as tests/test_attn_bwd.py:82-94
  backward  cuda/volta_mma_attn_bwd.cu:208-327 and the closed form tests/test_attn_bwd.py:95-101
  packed    cuda/volta_attn.h:39-52 (layout and gate), cuda/volta_mma_attn.cu:544-592,
            tests/test_packed_attention.py:40-57 (gated reference and trim_limits)
  trim      cuda/volta_mma_attn.cu:155-167, 258 (zero tiles past lims[N], keys up to lims[n])

Conventions the kernels share and this file keeps:
  * a masked key's logit is REPLACED by MASKED_LOGIT = -1e4 (its bias ignored), so an all-masked
    row is a uniform average, not a NaN (cuda/volta_attn.h:9-11);
  * lse is returned in the log2 domain, lse2 = log2(sum_k exp(logit_k)) (volta_mma_attn.cu:431-445);
  * a masked key has no gradient into its logit: dS = 0 there, but P still carries dV
    (volta_mma_attn_bwd.cu:218-228);
  * dbias is the fp32 sum of dS over the batch rows, unscaled (volta_mma_attn_bwd.cu:230-236).

Pinned by (tests/test_oracle_attention.py): torch float64 scaled_dot_product_attention with an
explicit scale for bias 0 / no mask; a brute-force per-element loop on tiny shapes; torch float64
autograd of an independent torch formulation for every gradient; central finite differences on
tiny shapes; the closed-form special cases (one key: out = v and zero gradients; an all-masked
row: uniform mean and lse2 = log2(Sk) - 1e4 * log2(e)); and the committed golden fixtures.
"""
import numpy as np
import torch

MASKED_LOGIT = -1.0e4
LOG2E = 1.4426950408889634


def _f64(*xs):
    """float64 CPU tensors: the dense products and elementwise passes run on torch's CPU
    kernels (all host cores), which is what lets the oracle cover BASELINE-sized problems."""
    return [torch.from_numpy(np.ascontiguousarray(x, dtype=np.float64)) for x in xs]


def _logits(q, k, bias, kmask, scale):
    """[N,H,Sq,Sk] natural-log-domain logits with the replace-mask convention."""
    m = torch.from_numpy(np.ascontiguousarray(np.asarray(kmask) != 0))[:, None, None, :]
    raw = scale * torch.matmul(q, k.transpose(-1, -2)) + bias[None]
    return torch.where(m, raw, torch.tensor(MASKED_LOGIT, dtype=torch.float64)), m


def attention_fwd(q, k, v, bias, kmask, scale):
    """out [N,H,Sq,D] and lse2 [N,H,Sq] (log2 domain) in float64.

    q [N,H,Sq,D], k/v [N,H,Sk,D], bias [H,Sq,Sk], kmask [N,Sk] (nonzero = keep).
    Follows tests/test_attn_bwd.py:82-94. Sk == 0 gives out 0 and lse2 -inf, as the kernel's
    empty key loop leaves l = 0 (volta_mma_attn.cu:441, 456).
    """
    q, k, v, bias = _f64(q, k, v, bias)
    n, h, sq, d = q.shape
    if k.shape[2] == 0:
        return np.zeros((n, h, sq, d)), np.full((n, h, sq), -np.inf)
    logits, _ = _logits(q, k, bias, kmask, scale)
    mx = logits.amax(-1, keepdim=True)
    e = torch.exp(logits - mx)
    l = e.sum(-1, keepdim=True)
    out = torch.matmul(e / l, v)
    lse2 = (torch.log(l) + mx)[..., 0] * LOG2E
    return out.numpy(), lse2.numpy()


def attention_bwd(q, k, v, bias, kmask, dout, scale):
    """dq, dk, dv [like q,k,v] and dbias [H,Sq,Sk] in float64 (tests/test_attn_bwd.py:95-101)."""
    q, k, v, bias, dout = _f64(q, k, v, bias, dout)
    if k.shape[2] == 0:
        h, sq = q.shape[1], q.shape[2]
        return (np.zeros(tuple(q.shape)), np.zeros(tuple(k.shape)), np.zeros(tuple(v.shape)),
                np.zeros((h, sq, 0)))
    logits, m = _logits(q, k, bias, kmask, scale)
    p = torch.softmax(logits, -1)
    dv = torch.matmul(p.transpose(-1, -2), dout)
    dp = torch.matmul(dout, v.transpose(-1, -2))
    ds = p * (dp - (p * dp).sum(-1, keepdim=True))
    ds = torch.where(m, ds, torch.zeros((), dtype=torch.float64))
    dq = torch.matmul(ds, k) * scale
    dk = torch.matmul(ds.transpose(-1, -2), q) * scale
    return dq.numpy(), dk.numpy(), dv.numpy(), ds.sum(0).numpy()


def attention_fwd_chunked(q, k, v, bias, kmask, scale, rows=8):
    """attention_fwd over batch-row chunks: identical math, bounded memory for large N."""
    outs, lses = [], []
    for n0 in range(0, q.shape[0], rows):
        o, l = attention_fwd(q[n0:n0 + rows], k[n0:n0 + rows], v[n0:n0 + rows], bias,
                             kmask[n0:n0 + rows], scale)
        outs.append(o)
        lses.append(l)
    return np.concatenate(outs), np.concatenate(lses)


def attention_bwd_chunked(q, k, v, bias, kmask, dout, scale, rows=8):
    """attention_bwd over batch-row chunks, dbias summed chunk by chunk."""
    dqs, dks, dvs, dbias = [], [], [], 0.0
    for n0 in range(0, q.shape[0], rows):
        s = slice(n0, n0 + rows)
        dq, dk, dv, db = attention_bwd(q[s], k[s], v[s], bias, kmask[s], dout[s], scale)
        dqs.append(dq)
        dks.append(dk)
        dvs.append(dv)
        dbias = dbias + db
    return np.concatenate(dqs), np.concatenate(dks), np.concatenate(dvs), dbias


def unpack(p, column):
    """q, k, v, gate as [N,H,S,D] from the packed projection p [X,Y,G,H,D].

    Rows (column False) attend along Y with batch X; columns along X with batch Y
    (cuda/volta_attn.h:39-45). gate is None when G == 3.
    """
    p = np.asarray(p, np.float64)
    if column:
        p = np.transpose(p, (1, 0, 2, 3, 4))
    # [N, S, G, H, D] -> per slot [N, H, S, D]
    slots = [np.transpose(p[:, :, i], (0, 2, 1, 3)) for i in range(p.shape[2])]
    gate = slots[3] if len(slots) == 4 else None
    return slots[0], slots[1], slots[2], gate


def repack_out(o, column):
    """[N,H,S,D] attention output -> out [X,Y,H,D] of the packed form."""
    o = np.transpose(o, (0, 2, 1, 3))  # [N, S, H, D]
    return np.transpose(o, (1, 0, 2, 3)) if column else o


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def trim_limits(kmask):
    """lims [N+1] int32: each batch row's last live key + 1 (0 if none), then the largest.

    tests/test_packed_attention.py:53-57.
    """
    kmask = np.asarray(kmask) != 0
    s = kmask.shape[1]
    last = np.where(kmask.any(axis=1), s - np.argmax(kmask[:, ::-1], axis=1), 0)
    return np.concatenate([last, [last.max() if last.size else 0]]).astype(np.int32)


def attention_packed(p, bias, kmask, gate_bias, column, scale=None, lims=None):
    """Gated packed forward, out [X,Y,H,D] float64 (tests/test_packed_attention.py:40-50).

    p [X,Y,G,H,D] with G in {3,4}; bias [H,S,S]; kmask [N,S]; gate_bias [H,D] (used when G == 4).
    With lims (trim), a batch row with lims[n] == 0 and every query at or past lims[N] is zero
    (the strict form of volta_mma_attn.cu:155-167), and keys stop at lims[n] (:258).
    """
    q, k, v, g = unpack(p, column)
    d = q.shape[-1]
    if scale is None:
        scale = d ** -0.5
    kmask = np.asarray(kmask)
    if lims is None:
        o, _ = attention_fwd(q, k, v, bias, kmask, scale)
    else:
        lims = np.asarray(lims)
        n_rows, s = kmask.shape
        o = np.zeros(q.shape)
        for n in range(n_rows):
            kend = int(lims[n])
            if kend == 0:
                continue
            on, _ = attention_fwd(q[n:n + 1], k[n:n + 1, :, :kend], v[n:n + 1, :, :kend],
                                  np.asarray(bias)[:, :, :kend], kmask[n:n + 1, :kend], scale)
            o[n] = on[0]
        o[:, :, int(lims[n_rows]):, :] = 0.0
    if g is not None:
        gb = np.asarray(gate_bias, np.float64).reshape(q.shape[1], d)
        o = o * sigmoid(g + gb[None, :, None, :])
        if lims is not None:
            o[:, :, int(lims[-1]):, :] = 0.0
            o[np.asarray(lims[:-1]) == 0] = 0.0
    return repack_out(o, column)

