"""Package metadata, and a build hook that compiles libgsvox.so (build.py:
hipcc for gfx950) before the package files are collected, so both regular and
editable installs carry the library next to gs_voxelizer/__init__.py."""
import importlib.util
import os

from setuptools import setup
from setuptools.command.build_py import build_py
from setuptools.dist import Distribution

HERE = os.path.dirname(os.path.abspath(__file__))


class BuildWithLibrary(build_py):
    def run(self):
        spec = importlib.util.spec_from_file_location("gsv_build", os.path.join(HERE, "build.py"))
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build(verbose=True)
        super().run()


class BinaryDistribution(Distribution):
    """The wheel carries a gfx950 shared library: tag it for the platform."""

    def has_ext_modules(self):
        return True


setup(
    name="gs-voxelizer-amd",
    version="0.2.0",
    description="MI355X-native (gfx950 HIP) drop-in for the gs_voxelizer Gaussian voxelizer",
    license="MIT",
    python_requires=">=3.9",
    packages=["gs_voxelizer"],
    package_data={"gs_voxelizer": ["libgsvox.so"]},
    install_requires=["torch", "numpy"],
    cmdclass={"build_py": BuildWithLibrary},
    distclass=BinaryDistribution,
)
