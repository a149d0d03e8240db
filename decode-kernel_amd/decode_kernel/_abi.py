"""ctypes view of the C ABI in include/decode_kernel/dk_gemv.h and dk_mlp.h.

This is the binding a non-torch host (or a maintainer wiring the library into
another runtime) would write: plain pointers, sizes and a hipStream_t handle.
The torch extension `decode_kernel._cuda` calls the same entry points from
C++. Loading the library needs no GPU; calling a compute entry point does.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libdk_hip.so"

DK_OK = 0
DK_ERR_INVALID_ARGUMENT = 1
DK_ERR_HIP = 2
DK_ERR_UNSUPPORTED = 3
DK_NOALLOC_SCRATCH_BYTES = 512 << 10  # include/decode_kernel/dk_gemv.h


class GemvConfig(ctypes.Structure):
    """Mirror of dk_gemv_config."""

    _fields_ = [
        ("version", ctypes.c_int),
        ("split_k", ctypes.c_int),
        ("reuse_weights", ctypes.c_int),
        ("warps_per_row", ctypes.c_int),
    ]


class LaunchInfo(ctypes.Structure):
    """Mirror of dk_launch_info (dk_gemv_describe)."""

    _fields_ = [
        ("kernel", ctypes.c_char * 512),
        ("grid", ctypes.c_uint * 3),
        ("block", ctypes.c_uint * 3),
        ("launches", ctypes.c_int),
    ]


# name -> (restype, argtypes); the export list checked against the header.
_P = ctypes.c_void_p
_SIGNATURES = {
    "dk_gemv_config_default": (None, [ctypes.POINTER(GemvConfig)]),
    "dk_gemv_workspace_bytes": (
        ctypes.c_size_t,
        [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.POINTER(GemvConfig)],
    ),
    "dk_gemv_validate": (
        ctypes.c_int,
        [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.POINTER(GemvConfig)],
    ),
    "dk_w4a16_gemv": (
        ctypes.c_int,
        [_P, _P, _P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int,
         ctypes.POINTER(GemvConfig), _P, ctypes.c_size_t, _P],
    ),
    "dk_w4a16_gemv_ref_workspace": (
        ctypes.c_int,
        [_P, _P, _P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int,
         ctypes.POINTER(GemvConfig), _P, _P],
    ),
    "dk_w4a16_gemv_noalloc": (
        ctypes.c_int,
        [_P, _P, _P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int,
         ctypes.POINTER(GemvConfig), _P],
    ),
    "dk_gemv_describe": (
        ctypes.c_int,
        [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.POINTER(GemvConfig), ctypes.c_size_t,
         ctypes.POINTER(LaunchInfo)],
    ),
    "dk_quantize_pack_f32": (ctypes.c_int, [_P, ctypes.c_int, ctypes.c_int, _P, _P, _P]),
    "dk_repack_paired": (ctypes.c_int, [_P, _P, ctypes.c_int, ctypes.c_int, _P]),
    "dk_unpack_paired": (ctypes.c_int, [_P, _P, ctypes.c_int, ctypes.c_int, _P]),
    "dk_w4a16_gemv_paired": (
        ctypes.c_int,
        [_P, _P, _P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P],
    ),
    "dk_gate_up_silu": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P],
    ),
    "dk_mlp_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "dk_mlp_decode": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _P, _P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P,
         ctypes.c_size_t, _P],
    ),
    "dk_d2d_copy": (ctypes.c_int, [_P, _P, ctypes.c_size_t, _P]),
    "dk_stream_read": (ctypes.c_int, [_P, _P, ctypes.c_size_t, ctypes.c_int, _P]),
    "dk_stream_write": (ctypes.c_int, [_P, ctypes.c_size_t, ctypes.c_int, _P]),
    "dk_stream_recommended_blocks": (ctypes.c_int, []),
    "dk_last_kernel_stamp": (ctypes.c_int, []),
    "dk_empty_kernel": (ctypes.c_int, [_P]),
    "dk_last_error": (ctypes.c_char_p, []),
    "dk_abi_version": (ctypes.c_int, []),
}

EXPORTS = tuple(_SIGNATURES)


class DkError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"status {status}: {message}")
        self.status = status


def load(path: Path | str = LIB_PATH) -> ctypes.CDLL:
    """Load libdk_hip.so and attach the signatures above."""
    lib = ctypes.CDLL(str(path))
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def default_config(lib: ctypes.CDLL, **overrides) -> GemvConfig:
    cfg = GemvConfig()
    lib.dk_gemv_config_default(ctypes.byref(cfg))
    for k, v in overrides.items():
        setattr(cfg, k, int(v))
    return cfg


def describe(lib: ctypes.CDLL, m: int, k: int, b: int, workspace_bytes: int | None = None,
             **config) -> dict:
    """The kernel dk_w4a16_gemv would launch for this call (dk_gemv_describe):
    demangled name, grid, workgroup size and number of launches. Needs no GPU.
    By default the call passes dk_gemv_workspace_bytes(), as the torch binding
    does."""
    cfg = default_config(lib, **config)
    if workspace_bytes is None:
        workspace_bytes = lib.dk_gemv_workspace_bytes(m, k, b, ctypes.byref(cfg))
    info = LaunchInfo()
    check(lib, lib.dk_gemv_describe(m, k, b, ctypes.byref(cfg), workspace_bytes,
                                    ctypes.byref(info)))
    return {"kernel": info.kernel.decode(), "grid": list(info.grid), "block": list(info.block),
            "launches": info.launches}


def check(lib: ctypes.CDLL, status: int) -> None:
    if status != DK_OK:
        raise DkError(status, lib.dk_last_error().decode())
