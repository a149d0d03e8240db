"""ctypes view of dk_bench/libdk_bench.so, the measurement-only kernels
(csrc/bench/dk_bench_kernels.hip): read-floor probes, the load-only ablation
of the streaming GEMV and its split-K form, the GPU wall-clock timestamps of
the benchmark timer and the shader-clock probe. None of it is part of the
product library or its C ABI."""

from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libdk_bench.so"

_P = ctypes.c_void_p
_I = ctypes.c_int
_SIGNATURES = {
    "dkb_read_probe": (_I, [_P, ctypes.c_size_t, _P, _I, _I, _I, _I, _P]),
    "dkb_v5": (_I, [_I, _I, _I, _I, _I, _P, _P, _P, _P, _I, _I, _P]),
    "dkb_v4s": (_I, [_I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _I, _I, _P]),
    "dkb_timestamp": (_I, [_P, _I, _P]),
    "dkb_clock_probe": (_I, [_P, _I, _I, _P]),
    "dkb_wall_clock_khz": (_I, []),
}
EXPORTS = tuple(_SIGNATURES)

_lib = None


def load(path: Path | str = LIB_PATH) -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not Path(path).exists():
            raise ImportError(f"{path} is not built; run `python decode-kernel_amd/build_ext.py`")
        lib = ctypes.CDLL(str(path))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what}: status {rc}")


def stream_handle():
    import torch

    return torch.cuda.current_stream().cuda_stream


def read_probe(src, partials, blocks: int, threads: int, loads: int, nt: bool) -> None:
    check(load().dkb_read_probe(src.data_ptr(), src.numel() * src.element_size(),
                                partials.data_ptr(), blocks, threads, loads, int(nt),
                                stream_handle()), "read probe")


def v5(math: int, shape: tuple, packed, scales, x, y) -> None:
    """Streaming GEMV (B = 1) with shape (R, U, W, prefetch); math 0 product,
    1 no decode, 2 loads only."""
    r, u, w, pf = shape
    m, k = packed.shape[0], packed.shape[1] * 8
    check(load().dkb_v5(math, r, u, w, int(pf), packed.data_ptr(), scales.data_ptr(), x.data_ptr(),
                        y.data_ptr(), m, k, stream_handle()), f"v5 {shape} math {math}")


def parse_v5_shape(kernel_name: str) -> tuple | None:
    """(R, U, W, prefetch) of a gemv_v5_lds kernel name at one batch row, as
    dk_gemv_describe reports it; None for any other kernel."""
    key = "gemv_v5_lds<"
    if key not in kernel_name:
        return None
    args = [a.strip() for a in kernel_name.split(key, 1)[1].split(">", 1)[0].split(",")]
    r, u, w, nb = (int(a) for a in args[:4])
    if nb != 1:
        return None
    return (r, u, w, args[4] == "true")


def timestamp(buf, slot: int) -> None:
    """Write the GPU wall clock to buf[slot] (int64 tensor) on the current stream."""
    check(load().dkb_timestamp(buf.data_ptr(), slot, stream_handle()), "timestamp")


def wall_clock_khz() -> int:
    return int(load().dkb_wall_clock_khz())


def sclk_mhz(iters: int = 200000, blocks: int = 1) -> float:
    """The shader clock in MHz, from the clock probe kernel: SCLK cycles
    (s_memtime) over wall-clock ticks (s_memrealtime) across a spin of
    `iters` dependent steps in `blocks` one-wave workgroups."""
    import torch

    out = torch.zeros(5, dtype=torch.int64, device="cuda")
    check(load().dkb_clock_probe(out.data_ptr(), iters, blocks, stream_handle()), "clock probe")
    c0, c1, w0, w1, _ = (int(v) for v in out.cpu())
    return (c1 - c0) / (w1 - w0) * wall_clock_khz() / 1e3


def v4s(shape: tuple, packed, scales, x, y, math: int = 0) -> int:
    """The product's split-K kernel (B = 1) at shape (R, U, W, S, prefetch):
    R rows per wave, U chunks per lane per stage and slice, W waves per
    workgroup, S waves per row; math 0 product, 1 no decode, 2 loads only,
    at the shapes the v5 dispatch takes it for. Returns 3 (nothing launched)
    for a shape not instantiated in the measurement library."""
    r, u, w, s_, pf = shape
    m, k = packed.shape[0], packed.shape[1] * 8
    rc = load().dkb_v4s(math, r, u, w, s_, int(pf), packed.data_ptr(), scales.data_ptr(),
                        x.data_ptr(), y.data_ptr(), m, k, stream_handle())
    if rc not in (0, 3):
        raise RuntimeError(f"v4 split {shape} math {math}: status {rc}")
    return rc


def parse_kernel(kernel_name: str) -> tuple | None:
    """("v5", (R, U, W, prefetch)) for a gemv_v5_lds kernel name at one batch
    row, ("split", (R, U, W, S, prefetch)) for a gemv_v4_split one, as
    dk_gemv_describe reports them; None for any other kernel."""
    v5 = parse_v5_shape(kernel_name)
    if v5 is not None:
        return ("v5", v5)
    key = "gemv_v4_split<"
    if key not in kernel_name:
        return None
    args = [a.strip() for a in kernel_name.split(key, 1)[1].split(">", 1)[0].split(",")]
    r, u, w, s_, nb = (int(a) for a in args[:5])
    if nb != 1:
        return None
    return ("split", (r, u, w, s_, args[5] == "true"))


def run_kernel(kernel: tuple, math: int, packed, scales, x, y) -> None:
    """Launches a kernel parsed by parse_kernel with the given math (0
    product, 1 no decode, 2 loads only)."""
    kind, shape = kernel
    if kind == "v5":
        v5(math, shape, packed, scales, x, y)
    elif v4s(shape, packed, scales, x, y, math) == 3:
        raise RuntimeError(f"split {shape} math {math} is not in the measurement library")
