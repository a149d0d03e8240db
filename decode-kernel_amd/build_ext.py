"""In-tree build of the gfx950 kernel library and the torch extension.

    python decode-kernel_amd/build_ext.py            # build everything
    python decode-kernel_amd/build_ext.py --asm      # also write device asm

Outputs (next to the Python package so they travel with the source tree):
    decode_kernel/libdk_hip.so   hipcc --offload-arch=gfx950: kernels + C ABI
    decode_kernel/_cuda*.so      g++: pybind/torch binding linked to libdk_hip.so
    dk_bench/libdk_bench.so      hipcc: measurement-only kernels (not the product)
    _build/*.s                   device assembly for inspection (with --asm)

Replaces the reference's nvcc CUDAExtension (setup.py:47-76). No hipify pass
runs: the kernels are HIP sources compiled directly for gfx950 and the
binding uses the c10::hip stream API.
"""

from __future__ import annotations

import argparse
import os
import shlex
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent          # decode-kernel_amd/
REPO_ROOT = PKG_ROOT.parent
CSRC = PKG_ROOT / "csrc"
PKG = PKG_ROOT / "decode_kernel"
INCLUDE = REPO_ROOT / "include"
BUILD = PKG_ROOT / "_build"

ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
ARCH = os.environ.get("DK_OFFLOAD_ARCH", "gfx950")

HIP_SOURCES = [CSRC / "dk_gemv.hip", CSRC / "dk_stream.hip", CSRC / "dk_quant.hip"]
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Packed FP32 instructions are disabled for every kernel on this target.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Kernel arguments preloaded into SGPRs at wave launch (gfx950 supports
    # it; the compiler adds a prologue that loads them on firmware without
    # it). A v5 wave then issues its first HBM load without waiting on a
    # scalar load of its arguments: 2.5% at M = K = 4096.
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wall",
    "-Wno-unused-command-line-argument",
]

LIB = PKG / "libdk_hip.so"
# Measurement-only kernels (read-floor probes, the load-only ablation, the
# one-stage and split-K shape variants): dk_bench/libdk_bench.so, never
# linked into the product library.
BENCH_SOURCES = [CSRC / "bench" / "dk_bench_kernels.hip"]
BENCH_LIB = PKG_ROOT / "dk_bench" / "libdk_bench.so"


def ext_path() -> Path:
    return PKG / ("_cuda" + sysconfig.get_config_var("EXT_SUFFIX"))


def _run(cmd: list[str], quiet_warning: str | None = None) -> None:
    print("+", " ".join(shlex.quote(c) for c in cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    out = (proc.stdout or "") + (proc.stderr or "")
    lines = [ln for ln in out.splitlines() if not (quiet_warning and quiet_warning in ln)]
    if lines:
        print("\n".join(lines), flush=True)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {cmd[0]}")


def hipcc() -> str:
    return str(ROCM / "bin" / "hipcc")


def build_lib() -> Path:
    tmp = LIB.with_suffix(".so.tmp")
    _run([hipcc(), *HIP_FLAGS, "-shared", f"-I{INCLUDE}", f"-I{CSRC}",
          *map(str, HIP_SOURCES), "-o", str(tmp)],
         quiet_warning="packed-fp32-ops' is not a recognized feature")
    os.replace(tmp, LIB)
    return LIB


def build_bench_lib() -> Path:
    tmp = BENCH_LIB.with_suffix(".so.tmp")
    _run([hipcc(), *HIP_FLAGS, "-fvisibility=hidden", "-shared", f"-I{INCLUDE}", f"-I{CSRC}",
          *map(str, BENCH_SOURCES), "-o", str(tmp)],
         quiet_warning="packed-fp32-ops' is not a recognized feature")
    os.replace(tmp, BENCH_LIB)
    return BENCH_LIB


def build_asm() -> list[Path]:
    BUILD.mkdir(exist_ok=True)
    outs = []
    for src in HIP_SOURCES:
        out = BUILD / (src.stem + f"-{ARCH}.s")
        _run([hipcc(), *HIP_FLAGS, "--cuda-device-only", "-S", f"-I{INCLUDE}", f"-I{CSRC}",
              str(src), "-o", str(out)],
             quiet_warning="packed-fp32-ops' is not a recognized feature")
        outs.append(out)
    return outs


def build_binding() -> Path:
    import torch
    from torch.utils import cpp_extension

    out = ext_path()
    tmp = out.with_name(out.name + ".tmp")
    torch_lib = Path(cpp_extension.library_paths()[0])
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [
        os.environ.get("CXX", "g++"),
        "-O2", "-std=c++17", "-fPIC", "-shared",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        "-DTORCH_EXTENSION_NAME=_cuda",
        "-DTORCH_API_INCLUDE_EXTENSION_H",
        "-D__HIP_PLATFORM_AMD__=1",
        "-DUSE_ROCM=1",
        f"-I{INCLUDE}",
        *[f"-I{p}" for p in cpp_extension.include_paths()],
        f"-I{sysconfig.get_paths()['include']}",
        f"-I{ROCM / 'include'}",
        str(CSRC / "bindings.cpp"),
        "-o", str(tmp),
        f"-L{PKG}", "-ldk_hip",
        f"-L{torch_lib}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
        "-ltorch_python",
        "-Wl,-rpath,$ORIGIN",
        f"-Wl,-rpath,{torch_lib}",
    ]
    _run(cmd)
    os.replace(tmp, out)
    return out


def build(asm: bool = False) -> None:
    build_lib()
    build_binding()
    build_bench_lib()
    if asm:
        build_asm()


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--asm", action="store_true", help="also write device assembly to _build/")
    ap.add_argument("--lib-only", action="store_true", help="only build libdk_hip.so")
    ap.add_argument("--bench-only", action="store_true", help="only build dk_bench/libdk_bench.so")
    args = ap.parse_args()
    if args.lib_only:
        build_lib()
    elif args.bench_only:
        build_bench_lib()
    else:
        build(asm=args.asm)
    return 0


if __name__ == "__main__":
    sys.exit(main())
