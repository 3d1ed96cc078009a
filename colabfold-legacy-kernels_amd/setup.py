"""Wheel packaging of the prebuilt gfx950 library (build it first: python build.py).

The wheel carries kernels/gfx950/libcolabfold_gfx950.so as package data. It holds no Python
extension module, only a library that ctypes / XLA load, so the tag is py3-none-<platform>:
any CPython 3 on that platform, but not a pure wheel.
"""
from setuptools import setup
from setuptools.command.install import install
from setuptools.dist import Distribution

try:
    from setuptools.command.bdist_wheel import bdist_wheel
except ImportError:  # setuptools < 70
    from wheel.bdist_wheel import bdist_wheel


class PlatformWheel(bdist_wheel):
    def finalize_options(self):
        super().finalize_options()
        self.root_is_pure = False  # platform-specific: it ships a shared library

    def get_tag(self):
        plat = super().get_tag()[2]
        return "py3", "none", plat


class WithLibrary(Distribution):
    def has_ext_modules(self):
        return True


class InstallPlatlib(install):
    def finalize_options(self):
        super().finalize_options()
        self.install_lib = self.install_platlib  # the package sits at the wheel's root


setup(distclass=WithLibrary, cmdclass={"bdist_wheel": PlatformWheel, "install": InstallPlatlib})
