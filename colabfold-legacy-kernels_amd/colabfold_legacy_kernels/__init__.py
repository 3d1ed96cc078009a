"""ColabFold legacy kernels for AMD Instinct MI355X (gfx950).

The locator surface is the reference package's (src/colabfold_legacy_kernels/__init__.py:1-126):
KERNELS, available, library_path, symbol, kernel_dir, supported_capabilities and _resolve, with
the same errors (KeyError for an unknown kernel, FileNotFoundError for a capability, library or
file that is missing). The capability key is the gfx target number: 950, or the string
"gfx950", which _resolve normalises to 950.

symbol() names each kernel's XLA FFI handler (VoltaMma, VoltaMmaBwd, VoltaLnProj, ...), which the
library exports under the reference's names (include/colabfold_gfx950_xla.h). Under them is a
plain C entry point per target (clk_attention_fwd, ...; include/colabfold_gfx950.h), which
colabfold_legacy_kernels.hip calls from PyTorch.
"""

from pathlib import Path

__all__ = [
    "KERNELS",
    "available",
    "kernel_dir",
    "library_path",
    "supported_capabilities",
    "symbol",
]

__version__ = "0.6.0+gfx950"

_KERNEL_DIR = Path(__file__).resolve().parent / "kernels"

_CAPABILITIES = (950,)

_LIB = "libcolabfold_gfx950.so"

# Each kernel lists its libraries from the highest capability first, as the reference's table
# does.
_TABLE = {
    "attention": ((950, _LIB, "VoltaMma"),),
    "attention_bwd": ((950, _LIB, "VoltaMmaBwd"),),
    "layer_norm": ((950, _LIB, "VoltaLayerNorm"),),
    "gated_dual_proj": ((950, _LIB, "VoltaGdp"),),
    "ln_gated_dual_proj": ((950, _LIB, "VoltaLnGdp"),),
    "trimul_epilogue": ((950, _LIB, "VoltaTrimulEpilogue"),),
    "ln_projection": ((950, _LIB, "VoltaLnProj"),),
    "output_projection": ((950, _LIB, "VoltaOutProj"),),
    "transition": ((950, _LIB, "VoltaTransition"),),
    "opm_update": ((950, _LIB, "VoltaOpmUpdate"),),
    "opm_outer": ((950, _LIB, "VoltaOpmOuter"),),
}

KERNELS = tuple(_TABLE)


def supported_capabilities():
    """The gfx target numbers this package ships libraries for."""
    return _CAPABILITIES


def _normalise(cc):
    if isinstance(cc, str) and cc.lower().startswith("gfx"):
        return int(cc[3:])
    return int(cc)


def _resolve(kernel, cc):
    """(cc, library file, FFI symbol) serving `kernel` at capability `cc`, None for the last two where
    nothing does; an unknown kernel name raises KeyError."""
    if kernel not in _TABLE:
        raise KeyError(
            "unknown kernel %r, expected one of %s" % (kernel, ", ".join(KERNELS)))
    cc = _normalise(cc)
    if cc not in _CAPABILITIES:
        return cc, None, None
    for min_cc, lib, sym in _TABLE[kernel]:
        if cc >= min_cc:
            return cc, lib, sym
    return cc, None, None


def kernel_dir(cc):
    """Directory that holds the libraries built for capability `cc`."""
    cc, _, _ = _resolve("attention", cc)
    return str(_KERNEL_DIR / ("gfx%d" % cc))


def library_path(kernel, cc):
    """Path to the shared library implementing `kernel` at capability `cc`."""
    cc, lib, _ = _resolve(kernel, cc)
    if lib is None:
        raise FileNotFoundError(
            "no %s kernel for gfx%d" % (kernel, cc))
    path = _KERNEL_DIR / ("gfx%d" % cc) / lib
    if not path.is_file():
        raise FileNotFoundError("%s is not in this package" % path)
    return str(path)


def symbol(kernel, cc):
    """XLA FFI handler name under which the library exports `kernel`."""
    cc, lib, sym = _resolve(kernel, cc)
    if sym is None:
        raise FileNotFoundError(
            "no %s kernel for gfx%d" % (kernel, cc))
    return sym


def available(cc, kernel=None):
    """True when `kernel` (or, with None, every kernel in KERNELS) has its library in place for `cc`."""
    names = KERNELS if kernel is None else (kernel,)
    for name in names:
        try:
            library_path(name, cc)
        except (FileNotFoundError, KeyError):
            return False
    return True
