"""Weight re-layouts between the callers' natural weight shapes and the FFI targets' layouts.

The reference's FFI targets take their weights transposed or blocked; the callers' wrappers
(colabfold_kernels.fused_ops, not part of the reference repository) re-lay them out before each
call. The target layouts are fixed by the reference's FFI comments and kernels:

  ln_gated_dual_proj  wp, wg [K, P] -> wpT, wgT [P, K]          (cuda/volta_fused_ffi.h:42-43)
  trimul_epilogue     wo [C, O] -> woT [O, C]; wg [CA, O] -> wgT [O, CA]   (volta_fused_ffi.h:82-91)
  ln_projection       w [slots, K, n] -> wT [slots n, K], slot major;
                      wb [K, heads] -> wbT [heads, K]            (volta_fused_ffi.h:135-136)
  output_projection   w [K, N] -> wT [N, K]                      (volta_fused_ffi.h:178)
  transition          w1 [C, H] -> w1T [H, C]; w2 [H, C] -> w2T [H/64][C][64] with
                      w2T[j][c][i] = w2[64 j + i][c]             (volta_fused_ffi.h:216-217)

Each function takes and returns torch tensors (any device) or numpy arrays, and returns a
contiguous result of the input's dtype.
"""

HIDDEN_CHUNK = 64  # rows of w2 per block of the transition's blocked layout


def _contig(x):
    if hasattr(x, "contiguous"):
        return x.contiguous()
    import numpy as np
    return np.ascontiguousarray(x)


def _t(x):
    """The 2-D transpose, contiguous."""
    if x.ndim != 2:
        raise ValueError("expected a 2-D weight, got shape %s" % (tuple(x.shape),))
    return _contig(x.T)


def proj_pair_T(wp, wg):
    """wp, wg [K, P] -> wpT, wgT [P, K] (ln_gated_dual_proj)."""
    return _t(wp), _t(wg)


def linear_T(w):
    """w [K, N] -> wT [N, K] (output_projection, trimul_epilogue's wo and wg, transition's w1)."""
    return _t(w)


def slot_major(w):
    """w [slots, K, n] -> wT [slots n, K], slot major: wT[s n + j, k] = w[s, k, j] (ln_projection)."""
    if w.ndim != 3:
        raise ValueError("expected w [slots, K, n], got shape %s" % (tuple(w.shape),))
    slots, k, n = w.shape
    if hasattr(w, "permute"):
        return w.permute(0, 2, 1).reshape(slots * n, k).contiguous()
    return _contig(w.transpose(0, 2, 1).reshape(slots * n, k))


def heads_T(wb):
    """wb [K, heads] -> wbT [heads, K] (ln_projection's head bias)."""
    return _t(wb)


def w2_blocked(w2):
    """w2 [H, C] -> w2T [H/64][C][64], w2T[j][c][i] = w2[64 j + i][c] (transition)."""
    if w2.ndim != 2 or w2.shape[0] % HIDDEN_CHUNK:
        raise ValueError("expected w2 [H, C] with H a multiple of 64, got shape %s" % (tuple(w2.shape),))
    h, c = w2.shape
    blocks = w2.reshape(h // HIDDEN_CHUNK, HIDDEN_CHUNK, c)
    if hasattr(blocks, "permute"):
        return blocks.permute(0, 2, 1).contiguous()
    return _contig(blocks.transpose(0, 2, 1))


def w2_unblocked(w2T):
    """The inverse of w2_blocked: [H/64][C][64] -> w2 [H, C]."""
    j, c, i = w2T.shape
    if hasattr(w2T, "permute"):
        return w2T.permute(0, 2, 1).reshape(j * i, c).contiguous()
    return _contig(w2T.transpose(0, 2, 1).reshape(j * i, c))
