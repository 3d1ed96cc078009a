"""pytest setup: the `gpu` marker, import paths and shared helpers for the parity tests."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "colabfold-legacy-kernels_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built library")


# (test, result, raw max |got - want|, abs excess beyond half an fp16 ulp, rel) of the tests that
# call record_error; printed as a table at the end of the session
ERRORS = []


def record_error(test, name, got, want, fp16_out=True):
    """Raw max-abs error, abs_excess and rel of one result, kept for the session summary."""
    got64, want64 = np.asarray(got, np.float64), np.asarray(want, np.float64)
    raw = float(np.abs(got64 - want64).max()) if got64.size else 0.0
    e = abs_excess(got64, want64, fp16_out)
    r = rel(got64, want64)
    ERRORS.append((test, name, raw, e, r))
    return raw, e, r


def pytest_terminal_summary(terminalreporter):
    if not ERRORS:
        return
    tr = terminalreporter
    tr.write_sep("-", "errors against the float64 oracle (raw max abs | beyond half an fp16 ulp | rel)")
    for test, name, raw, e, r in ERRORS:
        tr.write_line("%-34s %-6s raw %.3e  excess %.3e  rel %.3e" % (test, name, raw, e, r))


def gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:  # noqa: BLE001
        return False


@pytest.fixture(scope="session")
def hip():
    """The gfx950 front end; a GPU test without a GPU or without the library fails loudly."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("gpu test on a machine without a GPU")
    from colabfold_legacy_kernels import hip as h
    h.lib()
    return h


def ulp16(x):
    """One fp16 ulp at |x| (subnormal spacing below 2^-14)."""
    a = np.abs(np.asarray(x, np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -14)))
    return 2.0 ** (e - 10)


def ulp_bf16(x):
    """One bf16 ulp at |x| (8-bit significand)."""
    a = np.abs(np.asarray(x, np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -126)))
    return 2.0 ** (e - 7)


def rel(a, b):
    """The reference tests' error metric (tests/test_attn_bwd.py:104-111)."""
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    if not np.isfinite(a).all():
        return float("inf")
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-3)) if a.size else 0.0


def abs_excess(got, want, fp16_out=True, bf16_out=False):
    """max |got - want| beyond half an output ulp of want (the unavoidable output rounding):
    an fp16 ulp, or a bf16 ulp with bf16_out."""
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    if got.size == 0:
        return 0.0
    if not np.isfinite(got).all():
        return float("inf")
    err = np.abs(got - want)
    if bf16_out:
        err = err - 0.5 * ulp_bf16(want)
    elif fp16_out:
        err = err - 0.5 * ulp16(want)
    return float(max(err.max(), 0.0))
