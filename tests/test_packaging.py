"""Packaging of the gfx950 library, as the reference's CI checks its own
(.github/workflows/build-and-publish.yml:54-89, setup.py:13-25, pyproject.toml:33-34): the
library's direct dependencies are the HIP runtime and the C library only (libstdc++ and libgcc
linked statically), it exports only the C ABI and the FFI handlers, and a py3-none-<platform>
wheel built from the package installs and resolves every handler symbol. CPU only."""
import os
import shutil
import subprocess
import sys
import zipfile

import pytest

import colabfold_legacy_kernels as clk

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "colabfold-legacy-kernels_amd")
ALLOWED = ("libamdhip64.so", "libc.so", "libm.so", "libdl.so", "libpthread.so", "librt.so",
           "ld-linux-x86-64.so")


def lib_path():
    return clk.library_path("attention", 950)


def test_direct_dependencies():
    out = subprocess.run(["readelf", "-d", lib_path()], capture_output=True, text=True, check=True).stdout
    needed = [l.split("[")[1].rstrip("]") for l in out.splitlines() if "(NEEDED)" in l]
    assert any(n.startswith("libamdhip64.so") for n in needed), needed
    bad = [n for n in needed if not n.startswith(ALLOWED)]
    assert not bad, "unexpected dynamic dependencies: %s" % bad


def test_exported_symbols():
    out = subprocess.run(["nm", "-D", "--defined-only", lib_path()], capture_output=True, text=True,
                         check=True).stdout
    names = [l.split()[-1] for l in out.splitlines() if l.strip()]
    stray = [n for n in names if not (n.startswith("clk_") or n.startswith("Volta"))]
    assert not stray, stray[:10]
    for kernel in clk.KERNELS:
        assert clk.symbol(kernel, 950) in names


@pytest.fixture(scope="module")
def wheel(tmp_path_factory):
    work = tmp_path_factory.mktemp("wheel")
    src = work / "src"
    shutil.copytree(PKG, src, ignore=shutil.ignore_patterns("__pycache__", "build", "*.egg-info"))
    dist = work / "dist"
    r = subprocess.run([sys.executable, "-m", "pip", "wheel", "--no-deps", "--no-build-isolation",
                        "--no-index", "-w", str(dist), str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    wheels = list(dist.glob("*.whl"))
    assert len(wheels) == 1, wheels
    return wheels[0]


def test_wheel_tag_and_contents(wheel):
    assert wheel.name.endswith("-py3-none-linux_x86_64.whl"), wheel.name
    names = zipfile.ZipFile(wheel).namelist()
    assert "colabfold_legacy_kernels/kernels/gfx950/libcolabfold_gfx950.so" in names
    assert "colabfold_legacy_kernels/hip.py" in names


def test_installed_wheel_resolves_every_symbol(wheel, tmp_path):
    target = tmp_path / "site"
    r = subprocess.run([sys.executable, "-m", "pip", "install", "--no-deps", "--no-index", "--target",
                        str(target), str(wheel)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    probe = (
        "import ctypes, sys\n"
        "sys.path.insert(0, %r)\n"
        "import colabfold_legacy_kernels as clk\n"
        "assert clk.__file__.startswith(%r), clk.__file__\n"
        "assert clk.available(950) and clk.available('gfx950')\n"
        "for kernel in clk.KERNELS:\n"
        "    lib = ctypes.cdll.LoadLibrary(clk.library_path(kernel, 950))\n"
        "    getattr(lib, clk.symbol(kernel, 950))\n"
        "lib = ctypes.cdll.LoadLibrary(clk.library_path('attention', 950))\n"
        "for name in ('VoltaMmaPacked', 'VoltaMmaPackedTrim', 'clk_attention_fwd'):\n"
        "    getattr(lib, name)\n"
        "print('resolved', len(clk.KERNELS))\n" % (str(target), str(target)))
    r = subprocess.run([sys.executable, "-c", probe], capture_output=True, text=True, cwd=str(tmp_path))
    assert r.returncode == 0 and "resolved 11" in r.stdout, r.stdout + r.stderr
