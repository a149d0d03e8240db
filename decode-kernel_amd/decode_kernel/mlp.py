"""Llama-style MLP decode step on the W4A16 GEMV (SwiGLU: gate, up, down).

    h = fp16(silu(Wg x) * (Wu x))     one fused kernel (gate and up together)
    y = Wd h                          the v5 GEMV

Wg, Wu are [I, H] and Wd is [H, I], all in the package's int4 group-128
format. The reference has no MLP op; this is the step either side of its
`gemv` (python/decode_kernel/__init__.py:32-83) in a decoder, written so a
caller replaces three gemv calls and an elementwise SiLU*mul by one call.
Like `gemv`, it runs only through the HIP extension.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .quantize import quantize_and_pack

__all__ = ["QuantizedMLP", "gate_up_silu", "mlp_decode"]


def _ext():
    from . import _ext as ext

    return ext()


def _batch(x: torch.Tensor) -> tuple[torch.Tensor, bool]:
    return (x.unsqueeze(0), True) if x.dim() == 1 else (x, False)


def gate_up_silu(
    x: torch.Tensor,
    gate_packed: torch.Tensor,
    gate_scales: torch.Tensor,
    up_packed: torch.Tensor,
    up_scales: torch.Tensor,
) -> torch.Tensor:
    """h[B, I] = fp16(silu(Wg x) * (Wu x)), g and u accumulated in fp32."""
    xb, squeeze = _batch(x)
    h = _ext().gate_up_silu(gate_packed, gate_scales, up_packed, up_scales, xb)
    return h[0] if squeeze else h


def mlp_decode(
    x: torch.Tensor,
    gate_packed: torch.Tensor,
    gate_scales: torch.Tensor,
    up_packed: torch.Tensor,
    up_scales: torch.Tensor,
    down_packed: torch.Tensor,
    down_scales: torch.Tensor,
) -> torch.Tensor:
    """y[B, H] = Wd fp16(silu(Wg x) * (Wu x)) in two launches."""
    xb, squeeze = _batch(x)
    y = _ext().mlp_decode(gate_packed, gate_scales, up_packed, up_scales, down_packed,
                          down_scales, xb)
    return y[0] if squeeze else y


@dataclass
class QuantizedMLP:
    """The three quantized projections of one MLP block, ready for decode."""

    gate_packed: torch.Tensor
    gate_scales: torch.Tensor
    up_packed: torch.Tensor
    up_scales: torch.Tensor
    down_packed: torch.Tensor
    down_scales: torch.Tensor

    @classmethod
    def from_float(cls, w_gate: torch.Tensor, w_up: torch.Tensor,
                   w_down: torch.Tensor) -> "QuantizedMLP":
        """Quantize fp32 weights (gate/up [I, H], down [H, I]) on their device."""
        if w_gate.shape != w_up.shape or w_down.shape != w_gate.shape[::-1]:
            raise ValueError("expected gate, up [I, H] and down [H, I]")
        gp, gs = quantize_and_pack(w_gate)
        up, us = quantize_and_pack(w_up)
        dp, ds = quantize_and_pack(w_down)
        return cls(gp, gs, up, us, dp, ds)

    @property
    def intermediate_size(self) -> int:
        return int(self.gate_packed.shape[0])

    @property
    def hidden_size(self) -> int:
        return int(self.down_packed.shape[0])

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        return mlp_decode(x, self.gate_packed, self.gate_scales, self.up_packed, self.up_scales,
                          self.down_packed, self.down_scales)
