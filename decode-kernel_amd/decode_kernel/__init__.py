"""W4A16 decode GEMV for MI355X: 4-bit grouped weights, fp16 activations,
fused dequantisation in hand-written gfx950 HIP kernels.

Same op API as python/decode_kernel/__init__.py of the reference: `gemv`,
`w4a16_linear`, `quantize_and_pack`, `dequantize`, `GROUP_SIZE`,
`cuda_available`. The compute path is the `decode_kernel._cuda` extension
over the C ABI in include/decode_kernel/dk_gemv.h; there is no CPU fallback,
and calling `gemv` without the built extension raises ImportError.
`mlp_decode`, `gate_up_silu` and `QuantizedMLP` (decode_kernel.mlp) run a
Llama-style MLP decode step on the same kernels (include/decode_kernel/dk_mlp.h);
`repack_paired` / `gemv_paired` (decode_kernel.layout) use the kernel-native
paired weight layout.
"""

from __future__ import annotations

from typing import Optional

import torch

from .layout import gemv_paired, repack_paired, unpack_paired
from .mlp import QuantizedMLP, gate_up_silu, mlp_decode
from .quantize import GROUP_SIZE, dequantize, quantize_and_pack

__all__ = [
    "GROUP_SIZE",
    "QuantizedMLP",
    "cuda_available",
    "dequantize",
    "gate_up_silu",
    "gemv",
    "gemv_paired",
    "mlp_decode",
    "quantize_and_pack",
    "repack_paired",
    "unpack_paired",
    "w4a16_linear",
]


def cuda_available() -> bool:
    """True when a GPU is visible and the HIP extension imports."""
    if not torch.cuda.is_available():
        return False
    try:
        from . import _cuda  # noqa: F401
    except Exception:
        return False
    return True


def _ext():
    try:
        from . import _cuda
    except ImportError as exc:  # fail loudly: no fallback path exists
        raise ImportError(
            "decode_kernel._cuda is not built; run "
            "`python decode-kernel_amd/build_ext.py` (hipcc, gfx950)"
        ) from exc
    return _cuda


def gemv(
    packed: torch.Tensor,
    scales: torch.Tensor,
    x: torch.Tensor,
    version: int = 5,
    split_k: int = 4,
    reuse_weights: bool = False,
    warps_per_row: int = 1,
) -> torch.Tensor:
    """Y[B, M] = W_dequant[M, K] @ X[B, K]^T in one fused kernel.

    packed int32 [M, K/8], scales fp16 [M, K/128], x fp16 [B, K] or [K].
    Reference: python/decode_kernel/__init__.py:32-59.
    """
    ext = _ext()
    if x.dim() == 1:
        x = x.unsqueeze(0)
    return ext.w4a16_gemv(
        packed, scales, x, int(version), int(split_k), bool(reuse_weights), int(warps_per_row)
    )


def w4a16_linear(
    x: torch.Tensor,
    packed: torch.Tensor,
    scales: torch.Tensor,
    version: int = 5,
    split_k: Optional[int] = None,
    reuse_weights: Optional[bool] = None,
) -> torch.Tensor:
    """Drop-in for a quantized, bias-free F.linear.

    Defaults as in python/decode_kernel/__init__.py:62-83: split_k 4 only for
    v4, and the weight-reuse path whenever more than one batch row is given.
    """
    if split_k is None:
        split_k = 4 if version == 4 else 1
    if reuse_weights is None:
        reuse_weights = x.dim() == 2 and x.size(0) > 1
    return gemv(
        packed,
        scales,
        x,
        version=version,
        split_k=split_k,
        reuse_weights=reuse_weights,
        warps_per_row=1,
    )
