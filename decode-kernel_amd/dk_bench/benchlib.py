"""ctypes view of dk_bench/libdk_bench.so, the measurement-only kernels
(csrc/bench/dk_bench_kernels.hip): read-floor probes, the load-only ablation
of the streaming GEMV, one-stage GEMV variants and split-K shape instances.
None of it is part of the product library or its C ABI."""

from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libdk_bench.so"

_P = ctypes.c_void_p
_I = ctypes.c_int
_SIGNATURES = {
    "dkb_read_probe": (_I, [_P, ctypes.c_size_t, _P, _I, _I, _I, _I, _P]),
    "dkb_v5": (_I, [_I, _I, _I, _I, _I, _P, _P, _P, _P, _I, _I, _P]),
    "dkb_onestage": (_I, [_I, _I, _I, _I, _P, _P, _P, _P, _I, _I, _P]),
    "dkb_v4": (_I, [_I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, ctypes.c_ulonglong, _I, _I,
                    _P]),
    "dkb_v4s": (_I, [_I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _I, _I, _P]),
    "dkb_reuse": (_I, [_I, _I, _I, _I, _I, _P, _P, _P, _P, _I, _I, _I, _P]),
    "dkb_reuse_split_workspace": (ctypes.c_size_t, [_I, _I, _I, _I]),
    "dkb_reuse_split": (_I, [_I, _I, _I, _I, _P, _P, _P, _P, _P, _I, _I, _I, _P]),
    "dkb_gate_up": (_I, [_I, _I, _I, _P, _P, _P, _P, _P, _P, _I, _I, _I, _P]),
    "dkb_timestamp": (_I, [_P, _I, _P]),
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


def onestage(w: int, s: int, lds: bool, weights_first: bool, packed, scales, x, y) -> None:
    m, k = packed.shape[0], packed.shape[1] * 8
    check(load().dkb_onestage(w, s, int(lds), int(weights_first), packed.data_ptr(),
                              scales.data_ptr(), x.data_ptr(), y.data_ptr(), m, k,
                              stream_handle()), f"onestage W{w} S{s}")


def v4(shape: tuple, reduce: int, splits: int, packed, scales, x, y, ws, tickets, gen: int) -> None:
    """Split-K GEMV (B = 1), shape (R, U, W, prefetch); reduce 0 tickets (the
    product's), 2 partials only (no y)."""
    r, u, w, pf = shape
    m, k = packed.shape[0], packed.shape[1] * 8
    check(load().dkb_v4(r, u, w, int(pf), reduce, splits, packed.data_ptr(), scales.data_ptr(),
                        x.data_ptr(), y.data_ptr(), ws.data_ptr(), tickets.data_ptr(), gen, m, k,
                        stream_handle()), f"v4 {shape} S{splits}")


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


def v4s(shape: tuple, packed, scales, x, y, math: int = 0) -> int:
    """The product's split-K kernel (B = 1) at shape (R, U, W, S, prefetch):
    R rows per wave, U chunks per lane per stage and slice, W waves per
    workgroup, S waves per row; math 0 product, 1 no decode, 2 loads only.
    Returns 3 (nothing launched) for a shape not instantiated in the
    measurement library."""
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


def reuse(kind: int, ks: int, rt: int, sg: int, pairs: bool, packed, scales, x, y) -> int:
    """The reuse path's tile kernels: kind 0 gemv_reuse<KS, RT, SG, pairs>,
    kind 1 gemv_reuse_lds<KS, RT, pairs, SG>, kind 2 gemv_reuse_pf<KS, RT>
    (SG 2, pairs), kinds 3 and 4 gemv_reuse_pf<KS, RT, kXL> with 4 and 2 x
    loads per block (up to 8 and 4 batch rows). Returns 3 (nothing launched)
    for a shape not instantiated in the measurement library."""
    m, k = packed.shape[0], packed.shape[1] * 8
    b = x.shape[0]
    rc = load().dkb_reuse(kind, ks, rt, sg, int(pairs), packed.data_ptr(), scales.data_ptr(),
                          x.data_ptr(), y.data_ptr(), m, k, b, stream_handle())
    if rc not in (0, 3):
        raise RuntimeError(f"reuse kind {kind} KS{ks} RT{rt} SG{sg}: status {rc}")
    return rc


def reuse_split_workspace(rt: int, s: int, m: int, b: int) -> int:
    """Bytes of the workspace reuse_split needs: tickets, then fp32 partials."""
    return int(load().dkb_reuse_split_workspace(rt, s, m, b))


def reuse_split(kind: int, ks: int, rt: int, s: int, packed, scales, x, y, workspace) -> int:
    """The split-K tile kernels, S slices per row: kind 0
    gemv_reuse_split<KS, RT, 2>, kind 1 gemv_reuse_split_pf<KS, RT>.
    workspace: a uint8 tensor of at least reuse_split_workspace() bytes.
    Returns 3 (nothing launched) for a shape not instantiated."""
    m, k = packed.shape[0], packed.shape[1] * 8
    b = x.shape[0]
    if workspace.numel() < reuse_split_workspace(rt, s, m, b):
        raise ValueError("workspace too small")
    rc = load().dkb_reuse_split(kind, ks, rt, s, packed.data_ptr(), scales.data_ptr(), x.data_ptr(),
                                y.data_ptr(), workspace.data_ptr(), m, k, b, stream_handle())
    if rc not in (0, 3):
        raise RuntimeError(f"reuse split kind {kind} KS{ks} RT{rt} S{s}: status {rc}")
    return rc


def gate_up(kind: int, ks: int, pairs: bool, gp, gs, up, us, x, h) -> int:
    """The fused gate/up tile kernels: kind 0 gate_up_silu_tiles<KS, 2,
    pairs>, kind 1 gate_up_silu_tiles_lds<KS, pairs>, kind 2
    gate_up_silu_tiles_pf<KS> (pairs), kind 3 gate_up_silu_tiles_pf<KS, 4>
    (up to 8 batch rows). Returns 3 (nothing launched) for a shape not
    instantiated in the measurement library."""
    i, hd = gp.shape[0], gp.shape[1] * 8
    b = x.shape[0]
    rc = load().dkb_gate_up(kind, ks, int(pairs), gp.data_ptr(), gs.data_ptr(), up.data_ptr(),
                            us.data_ptr(), x.data_ptr(), h.data_ptr(), i, hd, b, stream_handle())
    if rc not in (0, 3):
        raise RuntimeError(f"gate/up kind {kind} KS{ks}: status {rc}")
    return rc
