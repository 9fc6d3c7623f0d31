"""Installs this build under the reference's distribution name, hp_rms_norm
(the reference's setup.py:14,80-92: one package, torch as the only
requirement, the extension module ``_C`` inside it).

    pip install --no-build-isolation .

compiles the two product libraries in the source tree
(``hp_rms_norm_amd/build.py product``: libhprms.so with hipcc for gfx950,
``_C.so`` with g++ against the PyTorch-ROCm already installed, hence no
build isolation) and installs the packages ``hp_rms_norm_amd`` and its
import alias ``hp_rms_norm`` with them.  ``_C.so`` finds libhprms.so beside
itself (rpath $ORIGIN).  The bench library, the oracle and the tests are not
installed.  Working from the source tree needs no install: build with
``python hp_rms_norm_amd/build.py`` and put the tree on ``sys.path``.
"""
import os
import subprocess
import sys

from setuptools import setup
from setuptools.command.build_py import build_py
from setuptools.dist import Distribution

ROOT = os.path.dirname(os.path.abspath(__file__))


class BuildProductLibraries(build_py):
    def run(self):
        subprocess.check_call([sys.executable, os.path.join(ROOT, "hp_rms_norm_amd", "build.py"), "product"])
        super().run()


class BinaryDistribution(Distribution):
    """The wheel holds gfx950 and x86-64 binaries: tag it for this platform."""

    def has_ext_modules(self):
        return True


setup(
    name="hp_rms_norm",
    version="0.1.0",
    description="Fused residual-add + RMSNorm for AMD MI355X (gfx950)",
    packages=["hp_rms_norm_amd", "hp_rms_norm"],
    package_data={"hp_rms_norm_amd": ["libhprms.so", "_C.so"]},
    install_requires=["torch"],
    cmdclass={"build_py": BuildProductLibraries},
    distclass=BinaryDistribution,
    zip_safe=False,
)
