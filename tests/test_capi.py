"""The C ABI (include/colabfold_gfx950.h) on the CPU: the library loads, exports every declared
entry point and the reference's FFI target names, and rejects what the reference's handlers
reject, with their messages, before touching a device. No kernel is launched here."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "colabfold_gfx950.h")


@pytest.fixture(scope="module")
def lib():
    from colabfold_legacy_kernels import hip
    return hip.lib()


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\w[\w\s\*]*?\b(clk_\w+)\(", text, re.M)))


def test_every_declared_symbol_is_exported(lib):
    names = declared()
    assert "clk_attention_fwd" in names and "clk_transition" in names and len(names) >= 12
    for name in names:
        assert hasattr(lib, name), name


def test_version(lib):
    assert lib.clk_version().decode().startswith("0.6.0")


def _buffer_type():
    from colabfold_legacy_kernels import hip
    return hip.Buffer


FAKE = 0x100000  # never dereferenced: every call below fails validation first


def buf(dtype, *dims, data=FAKE):
    arr = (ctypes.c_int64 * max(len(dims), 1))(*dims)
    b = _buffer_type()(data, dtype, len(dims), arr)
    b._keep = arr
    return ctypes.byref(b), b


F16, F32, U8, S32 = 10, 11, 6, 4


def call_fwd(lib, q, k=None, lse_dims=None, d_cfg=(64, 32), want_lse=1, kdtype=F16):
    n, h, s, d = q
    k = k or (n, h, s, d)
    args = [buf(F16, *q), buf(kdtype, *k), buf(F16, *k), buf(F16, h, s, k[2]), buf(U8, n, k[2]),
            buf(F16, *q), buf(F32, *(lse_dims or (n, h, s)))]
    st = lib.clk_attention_fwd(None, 0, *[a[0] for a in args], ctypes.c_float(0.1), d_cfg[0], d_cfg[1], want_lse)
    return st, lib.clk_last_error().decode()


def test_forward_validation(lib):
    st, msg = call_fwd(lib, (2, 2, 8, 48), d_cfg=(64, 64))
    assert st == 3 and "unsupported (D, bq, bk)" in msg
    st, msg = call_fwd(lib, (2, 2, 8, 32), kdtype=F32)
    assert st == 3 and "must be F16" in msg
    st, msg = call_fwd(lib, (2, 2, 8, 32), lse_dims=(2, 2, 7))
    assert st == 3 and "lse" in msg
    # an empty batch succeeds without a launch
    st, msg = call_fwd(lib, (0, 2, 8, 32))
    assert st == 0 and msg == ""


def test_backward_validation(lib):
    n, h, s, d = 2, 2, 8, 32
    q = buf(F16, n, h, s, d)
    rest = [buf(F16, n, h, s, d), buf(F16, n, h, s, d), buf(F16, h, s, s), buf(U8, n, s), buf(F16, n, h, s, d),
            buf(F16, n, h, s, d), buf(F32, n, h, s + 1), buf(F16, n, h, s, d), buf(F16, n, h, s, d),
            buf(F16, n, h, s, d), buf(F32, h, s, s)]
    st = lib.clk_attention_bwd(None, 0, q[0], *[a[0] for a in rest], ctypes.c_float(0.1), 1, None, 0)
    assert st == 3 and "lse must be [N,H,Sq]" in lib.clk_last_error().decode()
    rest[6] = buf(F32, n, h, s)
    rest[10] = buf(F32, h, s, s + 1)
    st = lib.clk_attention_bwd(None, 0, q[0], *[a[0] for a in rest], ctypes.c_float(0.1), 1, None, 0)
    assert st == 3 and "bias and dbias must be [H,Sq,Sk]" in lib.clk_last_error().decode()


def test_fused_validation(lib):
    m = 100
    # ln_projection: K must be 64 or 128
    args = [buf(F16, m, 96), buf(F32, 96), buf(F32, 96), buf(F16, 64, 96), buf(F16, 4, 96), buf(F16, 1),
            buf(F16, m, 64), buf(F16, 4, m)]
    st = lib.clk_ln_projection(None, *[a[0] for a in args], ctypes.c_float(1e-5), 64, 4, 0)
    assert st == 3 and "K must be 64 or 128" in lib.clk_last_error().decode()
    # transition: H must be 2C or 4C
    args = [buf(F16, m, 128), buf(F32, 128), buf(F32, 128), buf(F16, 384, 128), buf(F16, 384),
            buf(F16, 384 * 128), buf(F16, 128), buf(F16, 1), buf(F16, m, 128)]
    st = lib.clk_transition(None, *[a[0] for a in args], ctypes.c_float(1e-5), 0, 0)
    assert st == 3 and "H 2C or 4C" in lib.clk_last_error().decode()
    # trimul epilogue: add_input needs O == CA
    args = [buf(F32, 64, m), buf(F16, m, 128), buf(F32, 128), buf(F32, 128), buf(F32, 64), buf(F32, 64),
            buf(F16, 64, 64), buf(F16, 64), buf(F16, 64, 128), buf(F16, 64), buf(F16, 1), buf(F16, m, 64)]
    st = lib.clk_trimul_epilogue(None, *[a[0] for a in args], ctypes.c_float(1e-5), 1, 0)
    assert st == 3 and "O == CA with add_input" in lib.clk_last_error().decode()
    # ln_gdp: P/2 must be 64 or 128
    args = [buf(F16, m, 64), buf(F32, 64), buf(F32, 64), buf(F16, 96, 64), buf(F16, 96), buf(F16, 96, 64),
            buf(F16, 96), buf(F16, m), buf(F16, 48, m), buf(F16, 48, m)]
    st = lib.clk_ln_gdp(None, *[a[0] for a in args], ctypes.c_float(1e-5))
    assert st == 3 and "P/2 must be 64 or 128" in lib.clk_last_error().decode()
    # output projection with M == 0 succeeds without a launch
    args = [buf(F16, 0, 64), buf(F16, 64, 64), buf(F16, 64), buf(F16, 1), buf(F16, 1), buf(F16, 0, 64)]
    assert lib.clk_output_projection(None, *[a[0] for a in args], 0, 0) == 0


def test_stage_hook_bounds(lib):
    assert lib.clk_set_stage_events(None, 0) == 0
    assert lib.clk_set_stage_events(None, 99) == 3


@pytest.mark.parametrize("n,h,sq,sk,d", [(0, 2, 24, 40, 32), (2, 2, 0, 40, 32), (2, 2, 24, 0, 32),
                                         (512, 8, 384, 384, 32), (3, 4, 70, 83, 16), (1, 1, 1, 1, 96)])
def test_backward_workspace_size(lib, n, h, sq, sk, d):
    """The workspace holds delta and lse2 (fp32, padded to 32 queries), the fp16 transposed bias
    (keys padded to 64) and the dBias partials: never less than those arrays, also for empty
    problems."""
    q, _ = buf(F16, n, h, sq, d)
    k, _ = buf(F16, n, h, sk, d)
    size = lib.clk_attention_bwd_workspace_size(0, q, k)
    sqa, ska = -(-sq // 32) * 32, -(-sk // 64) * 64
    assert size >= 4 * 2 * n * h * sqa + 2 * h * ska * sqa
    assert size % 256 == 0


def test_fused_activation_dtypes(lib):
    """The fused entry points take BF16 activations as a whole: x and every activation result
    BF16 together, weights and biases still F16; a mix is rejected before any launch."""
    BF16 = 16
    m = 100
    # transition: x BF16, out F16 -> rejected
    args = [buf(BF16, m, 128), buf(F32, 128), buf(F32, 128), buf(F16, 512, 128), buf(F16, 512),
            buf(F16, 512 * 128), buf(F16, 128), buf(F16, 1), buf(F16, m, 128)]
    st = lib.clk_transition(None, *[a[0] for a in args], ctypes.c_float(1e-5), 0, 0)
    assert st == 3 and "must be BF16" in lib.clk_last_error().decode()
    # transition: a BF16 weight is rejected as well
    args = [buf(BF16, m, 128), buf(F32, 128), buf(F32, 128), buf(BF16, 512, 128), buf(F16, 512),
            buf(F16, 512 * 128), buf(F16, 128), buf(F16, 1), buf(BF16, m, 128)]
    st = lib.clk_transition(None, *[a[0] for a in args], ctypes.c_float(1e-5), 0, 0)
    assert st == 3 and "must be F16" in lib.clk_last_error().decode()
    # output projection: BF16 o and out with an F16 residual -> rejected
    args = [buf(BF16, m, 64), buf(F16, 64, 64), buf(F16, 64), buf(F16, m, 64), buf(F16, 1),
            buf(BF16, m, 64)]
    st = lib.clk_output_projection(None, *[a[0] for a in args], 1, 0)
    assert st == 3 and "must be BF16" in lib.clk_last_error().decode()
    # all-BF16 activations with M == 0 pass validation and launch nothing
    args = [buf(BF16, 0, 64), buf(F16, 64, 64), buf(F16, 64), buf(BF16, 1), buf(F16, 1), buf(BF16, 0, 64)]
    assert lib.clk_output_projection(None, *[a[0] for a in args], 0, 0) == 0
    # ln_gdp: BF16 x with F16 left/right -> rejected
    args = [buf(BF16, m, 64), buf(F32, 64), buf(F32, 64), buf(F16, 128, 64), buf(F16, 128),
            buf(F16, 128, 64), buf(F16, 128), buf(F16, m), buf(F16, 64, m), buf(F16, 64, m)]
    st = lib.clk_ln_gdp(None, *[a[0] for a in args], ctypes.c_float(1e-5))
    assert st == 3 and "must be BF16" in lib.clk_last_error().decode()
