"""Symmetric grouped int4 weight format (group 128), the layout the kernels read.

Format (identical to python/decode_kernel/quantize.py:1-15 of the reference):

* every 128 consecutive weights of a row share one fp16 scale
  ``scale = max(|w|)/7`` (computed in fp32, clamped below at 1e-8, then
  rounded to fp16);
* ``q = clamp(round_half_even(w / scale_fp32), -7, 7)``, using the fp32 scale
  before its fp16 rounding;
* eight consecutive q are packed into one int32, weight ``k = 8*word + n`` in
  bits ``4n .. 4n+3`` as a two's-complement nibble (low nibble first).
  -8 (nibble 0x8) is a valid encoding the kernels decode, but this quantizer
  never produces it.

These functions run on whatever device the input tensor lives on; they are
the format producer, not the GEMV (which only exists as a HIP kernel). On a
GPU tensor with the default group size, quantize_and_pack runs the HIP
quantizer of the extension (bit-exact with the CPU path); other group sizes
use the torch formulation below on either device.
"""

from __future__ import annotations

import torch

GROUP_SIZE = 128
NIBBLES_PER_WORD = 8
QMIN, QMAX = -7, 7
SCALE_FLOOR = 1e-8

_NIBBLE_SHIFTS = tuple(range(0, 32, 4))


def _div_fp32(a: torch.Tensor, b) -> torch.Tensor:
    """Correctly rounded fp32 quotient a / b on any device.

    torch's GPU kernels divide by a Python scalar as a multiplication by its
    reciprocal, which can differ from IEEE fp32 division in the last bit and
    then flip a rounded weight. Dividing in float64 and rounding to fp32 gives
    the correctly rounded fp32 quotient (a double rounding 53 -> 24 bits is
    innocuous for division of fp32 operands), so CPU and GPU tensors quantize
    to the same bits.
    """
    den = b.double() if isinstance(b, torch.Tensor) else torch.tensor(
        float(b), dtype=torch.float64, device=a.device)
    return (a.double() / den).float()


def quantize_and_pack(
    weight: torch.Tensor, group_size: int = GROUP_SIZE
) -> tuple[torch.Tensor, torch.Tensor]:
    """W[M, K] -> (packed int32 [M, K/8], scales fp16 [M, K/group]).

    Reference: python/decode_kernel/quantize.py:26-51.
    """
    if weight.dim() != 2:
        raise ValueError("weight must be [M, K]")
    m, k = weight.shape
    if k % group_size != 0:
        raise ValueError(f"K={k} is not divisible by group_size={group_size}")
    if k % NIBBLES_PER_WORD != 0:
        raise ValueError(f"K={k} is not divisible by {NIBBLES_PER_WORD}")
    if weight.is_cuda and group_size == GROUP_SIZE:
        # Device tensors go through the HIP quantizer (one pass over W, no
        # temporaries); it needs the built extension like the GEMV does.
        from . import _cuda

        packed, scales = _cuda.quantize_and_pack(weight.float().contiguous())
        return packed, scales
    return quantize_and_pack_torch(weight, group_size)


def quantize_and_pack_torch(
    weight: torch.Tensor, group_size: int = GROUP_SIZE
) -> tuple[torch.Tensor, torch.Tensor]:
    """The quantizer as torch tensor arithmetic, on the input's device.

    Same result bits as the HIP quantizer; used for CPU tensors, other group
    sizes, and as the second formulation the GPU quantizer is checked against.
    """
    m, k = weight.shape
    if k % group_size != 0 or k % NIBBLES_PER_WORD != 0:
        raise ValueError(f"K={k} is not divisible by group_size={group_size} and 8")
    groups = weight.float().reshape(m, k // group_size, group_size)
    scale = _div_fp32(groups.abs().amax(dim=-1), float(QMAX)).clamp_min(SCALE_FLOOR)
    q = torch.round(_div_fp32(groups, scale[..., None])).clamp_(QMIN, QMAX).to(torch.int32)

    # Nibble fields are disjoint, so an int32 sum of the shifted fields is
    # their bitwise OR (the top field wraps to the sign bit, as intended).
    fields = (q.reshape(m, k // NIBBLES_PER_WORD, NIBBLES_PER_WORD) & 0xF) << torch.tensor(
        _NIBBLE_SHIFTS, dtype=torch.int32, device=q.device
    )
    packed = fields.sum(dim=-1, dtype=torch.int32)
    return packed.contiguous(), scale.half().contiguous()


def unpack_to_int(packed: torch.Tensor) -> torch.Tensor:
    """int32 words [M, K/8] -> signed q [M, K] in [-8, 7] (int32).

    Reference: python/decode_kernel/quantize.py:54-63.
    """
    m, words = packed.shape
    shifts = torch.tensor(_NIBBLE_SHIFTS, dtype=torch.int32, device=packed.device)
    nib = (packed.to(torch.int32)[..., None] >> shifts) & 0xF  # [M, words, 8]
    q = nib - ((nib & 0x8) << 1)  # two's complement of the 4-bit field
    return q.reshape(m, words * NIBBLES_PER_WORD).to(torch.int32)


def dequantize(
    packed: torch.Tensor,
    scales: torch.Tensor,
    group_size: int = GROUP_SIZE,
    dtype: torch.dtype = torch.float32,
) -> torch.Tensor:
    """Materialise W = q * scale [M, K] (for checks; the kernels never do this).

    Reference: python/decode_kernel/quantize.py:66-78.
    """
    q = unpack_to_int(packed).to(dtype)
    m, k = q.shape
    s = scales.to(dtype).reshape(m, k // group_size, 1)
    return (q.reshape(m, k // group_size, group_size) * s).reshape(m, k)
