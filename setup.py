"""pip install [-e] . for the MI355X decode-kernel build.

Builds the gfx950 kernel library (hipcc), the torch extension
decode_kernel._cuda (g++ against torch's headers) and the measurement-only
dk_bench/libdk_bench.so in place, through decode-kernel_amd/build_ext.py,
then installs the packages `decode_kernel` and `dk_bench` with them. Replaces
the reference's nvcc CUDAExtension (setup.py:47-76 there). Offline:
`pip install -e . --no-build-isolation` (torch comes from the environment).
DK_SKIP_HIP=1 installs the Python packages only (no compute path: `gemv`
then raises ImportError, as the reference's package does without nvcc).
"""

from __future__ import annotations

import importlib.util
import os
import sys
from pathlib import Path

from setuptools import setup
from setuptools.command.build_ext import build_ext
from setuptools.command.build_py import build_py

ROOT = Path(__file__).resolve().parent
PKG_ROOT = ROOT / "decode-kernel_amd"


def _build_native() -> None:
    if os.environ.get("DK_SKIP_HIP") == "1":
        print("decode-kernel: DK_SKIP_HIP=1, Python packages only", file=sys.stderr)
        return
    spec = importlib.util.spec_from_file_location("dk_build_ext", PKG_ROOT / "build_ext.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    mod.build()


class BuildPy(build_py):
    """Build the native libraries in place first, so they are package data."""

    def run(self):
        _build_native()
        super().run()


class BuildExt(build_ext):
    """Editable installs build in place; nothing else to compile here."""

    def run(self):
        if self.inplace:
            _build_native()


setup(
    name="decode-kernel-amd",
    version="0.2.0",
    description=("W4A16 fused-dequant decode GEMV for MI355X (gfx950): the decode_kernel op API "
                 "on hand-written HIP kernels"),
    python_requires=">=3.9",
    install_requires=["torch", "numpy"],
    extras_require={"dev": ["pytest", "pytest-timeout"]},
    package_dir={"": "decode-kernel_amd"},
    packages=["decode_kernel", "dk_bench"],
    package_data={"decode_kernel": ["*.so"], "dk_bench": ["*.so"]},
    cmdclass={"build_py": BuildPy, "build_ext": BuildExt},
)
