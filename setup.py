"""pip-installable drop-in for the reference's ``Laplace_subtraction_cuda`` extension.

``pip install .`` (or ``pip install --no-build-isolation .``) compiles the two
native libraries with this package's own hipcc / g++ steps (no hipify: the
sources are HIP) and installs

* the package ``laplacianformer_amd`` (Python API, ``liblfamd.so`` with the C ABI
  of ``include/laplacianformer_amd.h``, and the PyTorch extension), and
* ``Laplace_subtraction_cuda`` as a top-level extension module next to it: the
  module name and exports the reference's ``setup.py`` builds
  (reference ``setup.py:7-40``, ``src/wrapper.cpp:73-99``), so ``import
  Laplace_subtraction_cuda`` works unchanged in a model repository.
"""
import os
import shutil
import sys

from setuptools import setup
from setuptools.command.build_py import build_py
from setuptools.dist import Distribution

ROOT = os.path.dirname(os.path.abspath(__file__))


class BuildNative(build_py):
    """Builds (or reuses up-to-date) native libraries, then stages the
    top-level module beside the package."""

    def run(self):
        sys.path.insert(0, ROOT)
        from laplacianformer_amd import _build

        _build.build_if_stale(verbose=self.verbose > 1)
        super().run()
        os.makedirs(self.build_lib, exist_ok=True)
        shutil.copy2(_build.EXT_PATH, os.path.join(self.build_lib, _build.EXT_NAME + ".so"))


class BinaryDistribution(Distribution):
    def has_ext_modules(self):
        return True


setup(
    name="laplacianformer-amd",
    version="0.2.0",
    description="MI355X-native LaplaceSubtraction and NewtonInverse (drop-in Laplace_subtraction_cuda)",
    packages=["laplacianformer_amd"],
    package_data={"laplacianformer_amd": ["liblfamd.so", "Laplace_subtraction_cuda.so"]},
    cmdclass={"build_py": BuildNative},
    distclass=BinaryDistribution,
    python_requires=">=3.8",
    zip_safe=False,
)
