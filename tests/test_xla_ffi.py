"""The XLA FFI handler symbols (include/colabfold_gfx950_xla.h) on the CPU, driven through a mock
of the XLA API table: the metadata handshake reports API 0.1 and the reference's traits, stages
other than EXECUTE do nothing, the call frame is decoded with the reference's buffer and
attribute orders, and rejections come back as XLA errors with the C ABI's codes and messages.
No kernel is launched here (every call below is rejected before a launch)."""
import os
import re

import pytest

import ffi_frames as ff

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HANDLERS = ("VoltaMma", "VoltaMmaPacked", "VoltaMmaPackedTrim", "VoltaMmaBwd", "VoltaLnGdp",
            "VoltaTrimulEpilogue", "VoltaLnProj", "VoltaOutProj", "VoltaTransition",
            "VoltaLayerNorm", "VoltaGdp", "VoltaOpmUpdate", "VoltaOpmOuter")
FAKE = 0x100000  # never dereferenced


@pytest.fixture(scope="module")
def lib():
    from colabfold_legacy_kernels import hip
    return hip.lib()


def test_every_declared_handler_is_exported(lib):
    text = open(os.path.join(ROOT, "include", "colabfold_gfx950_xla.h")).read()
    declared = sorted(set(re.findall(r"XLA_FFI_Error\*\s+(\w+)\(", text)))
    assert declared == sorted(HANDLERS)
    for name in declared:
        assert hasattr(lib, name), name


def test_locator_symbols_are_handlers(lib):
    import colabfold_legacy_kernels as clk
    for kernel in clk.KERNELS:
        if clk.available(950, kernel):
            assert clk.symbol(kernel, 950) in HANDLERS
            assert hasattr(lib, clk.symbol(kernel, 950))


@pytest.mark.parametrize("name", HANDLERS)
def test_metadata(lib, name):
    major, minor, traits = ff.metadata(getattr(lib, name))
    assert (major, minor) == (0, 1)
    # every target is command-buffer compatible except the backward (volta_mma_attn_bwd.cu:453)
    assert traits == (0 if name == "VoltaMmaBwd" else 1)


@pytest.mark.parametrize("name", HANDLERS)
def test_non_execute_stages_do_nothing(lib, name):
    mock = ff.MockXla()
    for stage in (0, 1, 2):
        assert mock.call(getattr(lib, name), [], [], {}, stage=stage) is None
    assert not mock.errors and mock.stream_gets == 0


def fwd_frame(d=32, bq=64, bk=32, n=2, h=2, s=8, kdtype=ff.F16, drop=None, attr_types=None):
    args = [(ff.F16, FAKE, (n, h, s, d)), (kdtype, FAKE, (n, h, s, d)), (ff.F16, FAKE, (n, h, s, d)),
            (ff.F16, FAKE, (h, s, s)), (ff.U8, FAKE, (n, s))]
    rets = [(ff.F16, FAKE, (n, h, s, d)), (ff.F32, FAKE, (n, h, s))]
    attrs = {"scale": (ff.F32, 0.125), "block_q": (ff.S64, bq), "block_k": (ff.S64, bk),
             "want_lse": (ff.PRED, 1)}
    attrs.update(attr_types or {})
    if drop:
        attrs.pop(drop)
    return args, rets, attrs


def test_forward_decoding_errors(lib):
    mock = ff.MockXla()
    args, rets, attrs = fwd_frame()
    assert mock.call(lib.VoltaMma, args[:4], rets, attrs) is not None
    assert mock.errors[-1] == (ff.INVALID_ARGUMENT, "Wrong number of arguments: expected 5 but got 4")
    assert mock.call(lib.VoltaMma, args, rets[:1], attrs) is not None
    assert mock.errors[-1] == (ff.INVALID_ARGUMENT, "Wrong number of results: expected 2 but got 1")
    args, rets, attrs = fwd_frame(drop="want_lse")
    assert mock.call(lib.VoltaMma, args, rets, attrs) is not None
    assert mock.errors[-1] == (ff.INVALID_ARGUMENT, "missing attribute want_lse")
    args, rets, attrs = fwd_frame(attr_types={"scale": (ff.S64, 1)})
    assert mock.call(lib.VoltaMma, args, rets, attrs) is not None
    assert mock.errors[-1] == (ff.INVALID_ARGUMENT, "attribute scale must be a f32 scalar")
    assert mock.stream_gets == 0  # decoding fails before the stream is asked for


def test_forward_validation_through_handler(lib):
    mock = ff.MockXla()
    args, rets, attrs = fwd_frame(d=48, bq=64, bk=64)
    assert mock.call(lib.VoltaMma, args, rets, attrs) is not None
    assert mock.errors[-1] == (ff.INVALID_ARGUMENT, "volta_mma: unsupported (D, bq, bk)")
    args, rets, attrs = fwd_frame(kdtype=ff.F32)
    assert mock.call(lib.VoltaMma, args, rets, attrs) is not None
    assert mock.errors[-1][0] == ff.INVALID_ARGUMENT and "must be F16" in mock.errors[-1][1]
    # an empty batch succeeds without a launch
    args, rets, attrs = fwd_frame(n=0)
    assert mock.call(lib.VoltaMma, args, rets, attrs) is None
    assert mock.stream_gets == 3


def test_backward_scratch_is_allocated_and_freed(lib):
    n, h, s, d = 2, 2, 8, 32
    mock = ff.MockXla(allocate=lambda size, align: 0x200000)
    q = (ff.F16, FAKE, (n, h, s, d))
    args = [q, q, q, (ff.F16, FAKE, (h, s, s)), (ff.U8, FAKE, (n, s)), q, q, (ff.F32, FAKE, (n, h, s + 1))]
    rets = [q, q, q, (ff.F32, FAKE, (h, s, s))]
    attrs = {"scale": (ff.F32, 0.1), "want_dbias": (ff.PRED, 1)}
    assert mock.call(lib.VoltaMmaBwd, args, rets, attrs) is not None
    assert mock.errors[-1] == (ff.INVALID_ARGUMENT, "volta_mma_bwd: lse must be [N,H,Sq]")
    (size, align, ptr), = mock.allocations
    assert size > 0 and align == 256 and mock.frees == [(size, ptr)]


def test_backward_scratch_failure(lib):
    n, h, s, d = 2, 2, 8, 32
    mock = ff.MockXla(allocate=lambda size, align: None)
    q = (ff.F16, FAKE, (n, h, s, d))
    args = [q, q, q, (ff.F16, FAKE, (h, s, s)), (ff.U8, FAKE, (n, s)), q, q, (ff.F32, FAKE, (n, h, s))]
    rets = [q, q, q, (ff.F32, FAKE, (h, s, s))]
    res = mock.call(lib.VoltaMmaBwd, args, rets, {"scale": (ff.F32, 0.1), "want_dbias": (ff.PRED, 1)})
    assert res is not None and mock.errors[-1] == (ff.INTERNAL, "mock: out of memory")
    assert not mock.frees


def test_fused_validation_through_handlers(lib):
    m = 100
    mock = ff.MockXla()
    args = [(ff.F16, FAKE, (m, 96)), (ff.F32, FAKE, (96,)), (ff.F32, FAKE, (96,)), (ff.F16, FAKE, (64, 96)),
            (ff.F16, FAKE, (4, 96)), (ff.F16, FAKE, (1,))]
    rets = [(ff.F16, FAKE, (m, 64)), (ff.F16, FAKE, (4, m))]
    attrs = {"eps": (ff.F32, 1e-5), "n": (ff.S64, 64), "heads": (ff.S64, 4), "has_keep": (ff.PRED, 0)}
    assert mock.call(lib.VoltaLnProj, args, rets, attrs) is not None
    assert mock.errors[-1][0] == ff.INVALID_ARGUMENT and "K must be 64 or 128" in mock.errors[-1][1]
    # output projection with M == 0 succeeds without a launch
    args = [(ff.F16, FAKE, (0, 64)), (ff.F16, FAKE, (64, 64)), (ff.F16, FAKE, (64,)), (ff.F16, FAKE, (1,)),
            (ff.F16, FAKE, (1,))]
    rets = [(ff.F16, FAKE, (0, 64))]
    attrs = {"has_residual": (ff.PRED, 0), "has_keep": (ff.PRED, 0)}
    assert mock.call(lib.VoltaOutProj, args, rets, attrs) is None


def test_plain_ops_validation_through_handlers(lib):
    mock = ff.MockXla()
    x = (ff.F16, FAKE, (10, 64))
    w = (ff.F16, FAKE, (64, 36))
    b = (ff.F16, FAKE, (36,))
    args = [x, w, b, w, b, (ff.F16, FAKE, (10,))]
    assert mock.call(lib.VoltaGdp, args, [(ff.F16, FAKE, (10, 36))], {"activation": (ff.S64, 0)}) is not None
    assert mock.errors[-1] == (ff.INVALID_ARGUMENT, "gdp: N must be a multiple of 8")
    w = (ff.F16, FAKE, (64, 32))
    b = (ff.F16, FAKE, (32,))
    args = [x, w, b, w, b, (ff.F16, FAKE, (10,))]
    assert mock.call(lib.VoltaGdp, args, [(ff.F16, FAKE, (10, 32))], {"activation": (ff.S64, 2)}) is not None
    assert mock.errors[-1] == (ff.INVALID_ARGUMENT, "gdp: activation is 0 (sigmoid) or 1 (swish), got 2")
    args = [(ff.F16, FAKE, (10, 64, 2)), (ff.F32, FAKE, (64,)), (ff.F32, FAKE, (64,))]
    assert mock.call(lib.VoltaLayerNorm, args, [(ff.F16, FAKE, (10, 64, 2))], {"eps": (ff.F32, 1e-5)}) is not None
    assert mock.errors[-1] == (ff.INVALID_ARGUMENT, "x must be [M,C]")
    # an empty batch succeeds without a launch
    args = [(ff.F16, FAKE, (0, 64)), (ff.F32, FAKE, (64,)), (ff.F32, FAKE, (64,))]
    assert mock.call(lib.VoltaLayerNorm, args, [(ff.F16, FAKE, (0, 64))], {"eps": (ff.F32, 1e-5)}) is None


def test_opm_validation_through_handlers(lib):
    """The reference's messages (cuda/volta_fused_ffi.h:266-283, 304-318)."""
    mock = ff.MockXla()
    up_attrs = {"eps": (ff.F32, 1e-3), "has_residual": (ff.PRED, 0)}
    one = (ff.F16, FAKE, (1,))

    def up(b, k, d, f, t_k=None, norm=None, res=one, attrs=up_attrs):
        args = [(ff.F16, FAKE, (b, k)), (ff.F16, FAKE, (k if t_k is None else t_k, d, f)),
                (ff.F32, FAKE, (f,)), (ff.F32, FAKE, norm or (b, d)), res]
        return mock.call(lib.VoltaOpmUpdate, args, [(ff.F16, FAKE, (b, d, f))], attrs)

    assert up(4, 64, 8, 128, t_k=32) is not None
    assert mock.errors[-1] == (ff.INVALID_ARGUMENT, "opm_update: lhs must be [B,K] and t [K,D,F]")
    bad_shape = "opm_update: K must be a multiple of 32, F 16, 32, 64 or 128, D at most 65535"
    for b, k, d, f in ((4, 48, 8, 128), (4, 64, 8, 96), (4, 64, 65536, 16)):
        assert up(b, k, d, f) is not None
        assert mock.errors[-1] == (ff.INVALID_ARGUMENT, bad_shape)
    assert up(4, 64, 8, 128, norm=(4, 9)) is not None
    assert mock.errors[-1] == (ff.INVALID_ARGUMENT, "opm_update: shapes do not match")
    attrs = dict(up_attrs, has_residual=(ff.PRED, 1))
    assert up(4, 64, 8, 128, attrs=attrs) is not None  # a one-element residual with has_residual
    assert mock.errors[-1] == (ff.INVALID_ARGUMENT, "opm_update: shapes do not match")
    assert up(0, 64, 8, 128) is None  # B == 0: nothing to do

    def outer(rows, b, c, d, e, f, wk=None):
        args = [(ff.F16, FAKE, (rows, b, c)), (ff.F16, FAKE, (rows, d, e)),
                (ff.F16, FAKE, (f, c * e if wk is None else wk))]
        return mock.call(lib.VoltaOpmOuter, args, [(ff.F16, FAKE, (b, d, f))], {})

    assert outer(32, 8, 32, 8, 32, 128) is not None
    assert mock.errors[-1] == (ff.INVALID_ARGUMENT,
                               "opm_outer: left must be [16,B,C], right [16,D,E], wT [F,C*E]")
    bad_shape = "opm_outer: C a multiple of 16, E 32, D a multiple of 4, F 16, 32, 64 or 128"
    for c, d, e, f, wk in ((24, 8, 32, 128, None), (32, 8, 16, 128, None), (32, 6, 32, 128, None),
                           (32, 8, 32, 96, None), (32, 8, 32, 128, 512)):
        assert outer(16, 8, c, d, e, f, wk) is not None
        assert mock.errors[-1] == (ff.INVALID_ARGUMENT, bad_shape)
    assert outer(16, 0, 32, 8, 32, 128) is None  # B == 0: nothing to do
