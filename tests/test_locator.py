"""The Python locator keeps the reference's surface (src/colabfold_legacy_kernels/__init__.py:1-126)
with a gfx950 row. CPU only; needs the built library for the path checks."""
import os

import pytest

import colabfold_legacy_kernels as clk

BUILT = ("attention", "attention_bwd", "layer_norm", "gated_dual_proj", "ln_gated_dual_proj",
         "trimul_epilogue", "ln_projection", "output_projection", "transition", "opm_update",
         "opm_outer")
SYMBOLS = {"attention": "VoltaMma", "attention_bwd": "VoltaMmaBwd", "layer_norm": "VoltaLayerNorm",
           "gated_dual_proj": "VoltaGdp", "ln_gated_dual_proj": "VoltaLnGdp",
           "trimul_epilogue": "VoltaTrimulEpilogue", "ln_projection": "VoltaLnProj",
           "output_projection": "VoltaOutProj", "transition": "VoltaTransition",
           "opm_update": "VoltaOpmUpdate", "opm_outer": "VoltaOpmOuter"}


def test_kernel_names_match_the_reference():
    assert clk.KERNELS == ("attention", "attention_bwd", "layer_norm", "gated_dual_proj",
                           "ln_gated_dual_proj", "trimul_epilogue", "ln_projection",
                           "output_projection", "transition", "opm_update", "opm_outer")
    assert clk.supported_capabilities() == (950,)
    assert clk.__version__.startswith("0.6.0")


@pytest.mark.parametrize("kernel", BUILT)
def test_symbols_and_paths(kernel):
    assert clk.symbol(kernel, 950) == SYMBOLS[kernel]
    assert clk.symbol(kernel, "gfx950") == SYMBOLS[kernel]
    path = clk.library_path(kernel, 950)
    assert os.path.isfile(path) and path.endswith("gfx950/libcolabfold_gfx950.so")
    assert clk.available(950, kernel)


def test_errors_as_the_reference():
    with pytest.raises(KeyError):
        clk.symbol("no_such_kernel", 950)
    with pytest.raises(FileNotFoundError):
        clk.library_path("attention", 75)      # a capability this package does not hold
    with pytest.raises(FileNotFoundError):
        clk.symbol("opm_outer", 75)            # no row for that capability
    assert clk.available(950)                  # every kernel of the table is built
    assert not clk.available(70)
    assert not clk.available(950, "no_such_kernel")
    assert clk.kernel_dir(950).endswith(os.path.join("kernels", "gfx950"))
    assert clk._resolve("attention", "gfx950") == (950, "libcolabfold_gfx950.so", "VoltaMma")
