"""Build and install flash_attn_legacy for AMD Instinct MI355X (gfx950).

Replaces the reference's setup.py (setup.py:1-120), which compiles CUDA kernels with
nvcc through torch's CUDAExtension.  Here the HIP sources under csrc/ are compiled
by build.py (hipcc, --offload-arch=gfx950) into flash_attn_legacy/libfal_hip.so, a
plain C-ABI library that the package loads with ctypes; the library ships as package
data.  `pip install .` and `python setup.py build_py` both run the HIP build first.
"""

import os
import sys

from setuptools import find_packages, setup
from setuptools.command.build_py import build_py
from setuptools.dist import Distribution

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)


class BuildHip(build_py):
    """Compile libfal_hip.so before the Python files are collected."""

    def run(self):
        import build as hip_build
        print(hip_build.build(), flush=True)
        super().run()


class NativeDistribution(Distribution):
    """The wheel carries a gfx950 shared library: tag it for the platform."""

    def has_ext_modules(self):
        return True


setup(
    name="flash_attn_legacy",
    version="0.5.0",
    description="Exact FlashAttention-2 (fp16/bf16) for AMD Instinct MI355X (gfx950)",
    packages=find_packages(include=["flash_attn_legacy", "flash_attn_legacy.*"]),
    package_data={"flash_attn_legacy": ["libfal_hip.so"]},
    python_requires=">=3.8",
    install_requires=["torch>=1.12.0"],
    extras_require={"hf": ["transformers>=4.34"], "test": ["pytest"]},
    cmdclass={"build_py": BuildHip},
    distclass=NativeDistribution,
    zip_safe=False,
)
