"""Float64 oracle for the LayerNorm-fused pair-stack projections (TEST INFRASTRUCTURE ONLY).

Closed forms restated from the reference kernels (their epilogues and FFI comments):
  layer_norm         cuda/volta_gdp.h:207-240 (two-pass fp32 statistics, biased variance)
  ln_columns         cuda/volta_gdp.h:242-287 (the same over channel-major x_cm)
  ln_gdp             cuda/volta_fused_ffi.h:42-43, cuda/volta_ops.cu:361-393
  trimul_epilogue    cuda/volta_fused_ffi.h:91, cuda/volta_ops.cu:429-465
  ln_projection      cuda/volta_fused_ffi.h:135-136, cuda/volta_ops.cu:503-541, volta_gdp.h:288-332
  output_projection  cuda/volta_fused_ffi.h:178, cuda/volta_ops.cu:513-541 (LN = false)
  transition         cuda/volta_fused_ffi.h:216-217, cuda/volta_ops.cu:585-634
  layer_norm_onepass cuda/volta_ops.cu:27-57 (VoltaLayerNorm: one-pass statistics, var clamped at 0)
  gated_dual_proj    cuda/volta_ops.cu:97-187, volta_gdp.h:10-35 (VoltaGdp: wp, wg [K, N],
                     out = mask (x@wp + bp) act(x@wg + bg), act sigmoid or swish)
  keep / tile_work   cuda/volta_gdp.h:114-160 and the padding branches at volta_ops.cu:349-356,
                     422-428, 491-502, 578-584

Rounding points (round_mid=True, the default, applies them; False keeps every intermediate in
float64): the LayerNorm output is fp16 before its GEMM (volta_gdp.h:237, 283-284), the transition
hidden activation is fp16 (volta_ops.cu:602-604), and the head-bias dot reads the fp16 LN output
(volta_gdp.h:307-320). Every GEMM accumulates in fp32 in the kernels and in float64 here.

Pinned by (tests/test_oracle_fused.py): torch float64 layer_norm (both LN forms); numpy matmul against an
explicit per-element sum on tiny shapes; the transition's blocked w2T layout against a direct
gather; the keep rule against a brute-force per-row statement of the reference's tile decision;
and the committed golden fixtures.
"""
import numpy as np

# keep granularity of the reference (cuda/volta_gdp.h:40-41, volta_ops.cu:551-553): a row tile of
# 64, or 32 for the tri-mul epilogue and for the transition at 256 channels
ROWS = 64
EPI_ROWS = 32
HIDDEN_CHUNK = 64

COMPUTE, PADDING, SKIP = 0, 1, 2


def f16(x):
    return np.asarray(x, np.float64).astype(np.float16).astype(np.float64)


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def layer_norm(x, scale, offset, eps, round_mid=True):
    """LN over the last axis with two-pass statistics (cuda/volta_gdp.h:207-240)."""
    x = np.asarray(x, np.float64)
    mean = x.mean(-1, keepdims=True)
    v = x - mean
    var = (v * v).mean(-1, keepdims=True)
    y = v / np.sqrt(var + eps) * np.asarray(scale, np.float64) + np.asarray(offset, np.float64)
    return f16(y) if round_mid else y


def tile_work(keep, m, rows, other):
    """Per row tile of `rows`: COMPUTE if any keep > 0, else PADDING if any keep == 0 (rows at
    or past M read as `other`), else SKIP (cuda/volta_gdp.h:114-136). keep None: all COMPUTE."""
    tiles = (m + rows - 1) // rows
    if keep is None:
        return np.zeros(tiles, np.int64)
    kp = np.full(tiles * rows, float(other))
    kp[:m] = np.asarray(keep, np.float64).reshape(-1)
    kp = kp.reshape(tiles, rows)
    live = (kp > 0).any(1)
    zero = (kp == 0).any(1)
    return np.where(live, COMPUTE, np.where(zero, PADDING, SKIP))


def _apply_keep(out, work, rows, pad_value, axis0_rows=True):
    """Write `out` rows by tile decision: computed tiles keep their values, padding tiles take
    pad_value (None: unchanged, i.e. NaN marker for 'not written'), skipped tiles are NaN
    (not written). Returns the array the kernel's output buffer would hold, with NaN where the
    kernel leaves the caller's memory untouched."""
    out = np.array(out, np.float64, copy=True)
    m = out.shape[0] if axis0_rows else out.shape[1]
    for t, w in enumerate(work):
        sl = slice(t * rows, min((t + 1) * rows, m))
        if w == COMPUTE:
            continue
        val = np.nan if (w == SKIP or pad_value is None) else pad_value
        if axis0_rows:
            out[sl] = val
        else:
            out[:, sl] = val
    return out


def ln_gdp(x, scale, offset, wpT, bp, wgT, bg, mask, eps, round_mid=True):
    """left, right [P/2, M]: mask * (y@wp + bp) * sigmoid(y@wg + bg), y = LN(x), channel major.

    wpT, wgT [P, K]; bp, bg [P]; mask [M] (also the keep, with rows past M counting as 0).
    NaN marks columns the kernel does not write (skipped tiles).
    """
    y = layer_norm(x, scale, offset, eps, round_mid)
    pr = y @ np.asarray(wpT, np.float64).T + np.asarray(bp, np.float64)
    g = y @ np.asarray(wgT, np.float64).T + np.asarray(bg, np.float64)
    mv = np.maximum(np.asarray(mask, np.float64), 0.0)[:, None]
    res = (mv * pr * sigmoid(g)).T  # [P, M]
    work = tile_work(mask, x.shape[0], ROWS, 0.0)
    res = _apply_keep(res, work, ROWS, 0.0, axis0_rows=False)
    half = res.shape[0] // 2
    return res[:half], res[half:]


def trimul_epilogue(x_cm, x, in_scale, in_offset, ln_scale, ln_offset, woT, bo, wgT, bg, keep,
                    eps, add_input, round_mid=True):
    """out [M,O] = (LN(x_cm.T)@wo + bo) * sigmoid(LN_in(x)@wg + bg) [+ x]. keep None: no keep."""
    y = layer_norm(np.asarray(x_cm, np.float64).T, ln_scale, ln_offset, eps, round_mid)
    a = layer_norm(x, in_scale, in_offset, eps, round_mid)
    out = (y @ np.asarray(woT, np.float64).T + np.asarray(bo, np.float64)) * sigmoid(
        a @ np.asarray(wgT, np.float64).T + np.asarray(bg, np.float64))
    if add_input:
        out = out + np.asarray(x, np.float64)
    work = tile_work(keep, out.shape[0], EPI_ROWS, -1.0)
    # with add_input the output aliases x: a padding tile keeps x
    return _apply_keep(out, work, EPI_ROWS, None if add_input else 0.0)


def ln_projection(x, scale, offset, wT, wbT, keep, eps, round_mid=True):
    """p [M,n] = LN(x)@w (no bias term) and bias [heads, M] = (LN(x)@wb).T.

    wT [n, K] or None (n == 0), wbT [heads, K] or None (heads == 0); the missing result is None.
    """
    y = layer_norm(x, scale, offset, eps, round_mid)
    m = y.shape[0]
    work = tile_work(keep, m, ROWS, -1.0)
    p = None if wT is None else _apply_keep(y @ np.asarray(wT, np.float64).T, work, ROWS, 0.0)
    b = None
    if wbT is not None:
        hb = (y @ np.asarray(wbT, np.float64).T).T  # [heads, M]
        b = _apply_keep(hb, work, ROWS, 0.0, axis0_rows=False)
    return p, b


def output_projection(o, wT, b, residual, keep):
    """out [M,N] = o@w + b [+ residual]; with a residual the output aliases it."""
    out = np.asarray(o, np.float64) @ np.asarray(wT, np.float64).T + np.asarray(b, np.float64)
    if residual is not None:
        out = out + np.asarray(residual, np.float64)
    work = tile_work(keep, out.shape[0], ROWS, -1.0)
    return _apply_keep(out, work, ROWS, None if residual is not None else 0.0)


def w2_blocked(w2):
    """w2 [H, C] -> w2T [H/64][C][64], w2T[j][c][i] = w2[64 j + i][c] (volta_fused_ffi.h:216-217)."""
    w2 = np.asarray(w2)
    hid, c = w2.shape
    return np.ascontiguousarray(w2.reshape(hid // HIDDEN_CHUNK, HIDDEN_CHUNK, c).transpose(0, 2, 1))


def w2_unblocked(w2T):
    """Inverse of w2_blocked: [H/64][C][64] -> w2 [H, C]."""
    w2T = np.asarray(w2T)
    j, c, i = w2T.shape
    return np.ascontiguousarray(w2T.transpose(0, 2, 1).reshape(j * i, c))


def transition_rows(c):
    return EPI_ROWS if c > 128 else ROWS


def transition(x, scale, offset, w1T, b1, w2T, b2, keep, eps, add_input, round_mid=True):
    """out [M,C] = relu(LN(x)@w1 + b1)@w2 + b2 [+ x]; w1T [H,C], w2T blocked [H/64][C][64]."""
    y = layer_norm(x, scale, offset, eps, round_mid)
    hid = np.maximum(y @ np.asarray(w1T, np.float64).T + np.asarray(b1, np.float64), 0.0)
    if round_mid:
        hid = f16(hid)
    w2 = w2_unblocked(w2T).astype(np.float64)
    out = hid @ w2 + np.asarray(b2, np.float64)
    if add_input:
        out = out + np.asarray(x, np.float64)
    rows = transition_rows(np.asarray(x).shape[1])
    work = tile_work(keep, out.shape[0], rows, -1.0)
    return _apply_keep(out, work, rows, None if add_input else 0.0)


def layer_norm_onepass(x, scale, offset, eps):
    """VoltaLayerNorm over the last axis: mean = E[x], var = max(E[x^2] - mean^2, 0),
    rstd = 1/sqrt(var + eps) (cuda/volta_ops.cu:40-56), evaluated in float64."""
    x = np.asarray(x, np.float64)
    mean = x.mean(-1, keepdims=True)
    var = np.maximum((x * x).mean(-1, keepdims=True) - mean * mean, 0.0)
    return (x - mean) / np.sqrt(var + eps) * np.asarray(scale, np.float64) + np.asarray(offset, np.float64)


def gated_dual_proj(x, wp, bp, wg, bg, mask, activation):
    """VoltaGdp: out [M, N] = mask[m] (x@wp + bp) act(x@wg + bg) with wp, wg [K, N]; act is
    sigmoid (0) or swish, g sigmoid(g) (1) (cuda/volta_ops.cu:168-186, volta_gdp.h:13-19)."""
    x = np.asarray(x, np.float64)
    p = x @ np.asarray(wp, np.float64) + np.asarray(bp, np.float64)
    g = x @ np.asarray(wg, np.float64) + np.asarray(bg, np.float64)
    act = sigmoid(g) if activation == 0 else g * sigmoid(g)
    return np.asarray(mask, np.float64)[:, None] * p * act
