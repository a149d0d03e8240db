"""fp32 dequantize-then-matmul on the CPU, for users' own accuracy checks.

Same functions as python/decode_kernel/reference.py:17-30 of the reference,
kept so code written against it keeps importing. `gemv` never calls this:
the GEMV exists only as a HIP kernel and raises if the extension is absent.
This repository's parity tests check the kernels against the independent
restatement under oracle/ instead.
"""

from __future__ import annotations

import torch

from .quantize import dequantize


def linear_fp32(x: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """Y[B, M] = X @ W_dequant^T in fp32 on the CPU; x may be [K] or [B, K]."""
    w = dequantize(packed.cpu(), scales.cpu(), dtype=torch.float32)
    xv = x.detach().cpu().float()
    if xv.dim() == 1:
        xv = xv[None, :]
    return xv @ w.t()


def max_abs_err(y_kernel: torch.Tensor, y_ref: torch.Tensor) -> float:
    return float((y_kernel.float().cpu() - y_ref.float().cpu()).abs().max().item())
