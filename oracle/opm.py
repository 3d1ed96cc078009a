"""Float64 oracle for the outer product mean kernels (TEST INFRASTRUCTURE ONLY).

Restated from the reference kernels and their FFI comments:
  opm_update  cuda/volta_ops.cu:647-698 (epilogue 678-697), cuda/volta_fused_ffi.h:261-297:
              out[b, d, :] = (lhs[b] @ t[:, d, :] + bias) / (eps + norm[b, d]) [+ residual[b, d, :]]
  opm_outer   cuda/volta_ops.cu:711-786, cuda/volta_fused_ffi.h:299-335:
              out[b, d, f] = sum_c sum_e f16(sum_a left[a, b, c] right[a, d, e]) wT[f, c E + e]
              over the 16 rows a, E = 32

Rounding points: opm_outer rounds the per-channel outer product g to fp16 before the second
contraction (volta_ops.cu:765-769; the reference's own test restates it as `outer_f32`,
tests/test_opm.py:82-86); both kernels accumulate in fp32 (float64 here) and round the output to
fp16 once (volta_ops.cu:693, 783).

The reference's float32 references for these ops (`ref_opm_update`, `ref_opm_outer`) live in the
separate colabfold-kernels package that tests/test_opm.py imports from CK_SRC; it is not part of
the reference tree, so the pins below rest on the reference's kernels, its test's `outer_f32`
statement and mathematics.

Pinned by (tests/test_oracle_opm.py): per-element brute-force sums on tiny shapes; opm_update
with zero bias, unit norm and zero eps against numpy matmul, and with zero lhs against the
closed form bias / (eps + norm); opm_outer against the reference test's einsum statement of its
rounding; a case whose only difference between rounding g and not is fixed by hand; and the
identity between the two kernels (opm_update on lhs[b, (a, c)] = left[a, b, c] and
t[(a, c), d, f] = sum_e right[a, d, e] wT[f, c E + e] equals opm_outer without the rounding of g).
"""
import numpy as np

ROWS = 16
E = 32
WIDTHS = (16, 32, 64, 128)


def f16(x):
    return np.asarray(x, np.float64).astype(np.float16).astype(np.float64)


def opm_update(lhs, t, bias, norm, eps, residual=None):
    """volta_ops.cu:647-698. lhs [B, K], t [K, D, F], bias [F], norm [B, D], residual [B, D, F]."""
    lhs = np.asarray(lhs, np.float64)
    t = np.asarray(t, np.float64)
    B, K = lhs.shape
    _, D, F = t.shape
    acc = (lhs @ t.reshape(K, D * F)).reshape(B, D, F)  # fp32 MMA accumulation
    out = (acc + np.asarray(bias, np.float64)[None, None, :]) / (
        eps + np.asarray(norm, np.float64)[:, :, None])
    if residual is not None:
        out = out + np.asarray(residual, np.float64)
    return out


def opm_outer(left, right, wT, round_mid=True):
    """volta_ops.cu:711-786, channel by channel as the kernel walks c. left [16, B, C],
    right [16, D, 32], wT [F, 32 C]."""
    left = np.asarray(left, np.float64)
    right = np.asarray(right, np.float64)
    wT = np.asarray(wT, np.float64)
    _, B, C = left.shape
    D = right.shape[1]
    F = wT.shape[0]
    out = np.zeros((B, D, F))
    for c in range(C):
        g = np.einsum("ab,ade->bde", left[:, :, c], right)  # [B, D, E], sum over the 16 rows
        if round_mid:
            g = f16(g)
        out += g @ wT[:, c * E:(c + 1) * E].T  # [B, D, E] @ [E, F]
    return out
