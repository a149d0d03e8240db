"""Kernel-native "paired" weight layout (an offline repack of the API format).

The API format (python/decode_kernel/quantize.py:1-15 of the reference) puts
nibble n of a word at bits 4n. The gfx950 decode turns nibbles 16 bits apart
into one fp16 pair, so with that order the pairs are (q0,q4), (q1,q5), ...
and eight activations must be permuted to match. The paired layout stores
the same two's-complement nibbles with q_{2j} at bits 4j and q_{2j+1} at
bits 16+4j, so the decoded pairs are (q0,q1), (q2,q3), ... and the
activations' natural fp16 pairs are used as loaded. Scales are unchanged.

    paired = repack_paired(packed)        # once, offline or at load time
    y = gemv_paired(paired, scales, x)    # the v5 GEMV, stamp 25
    assert torch.equal(unpack_paired(paired), packed)
"""

from __future__ import annotations

import torch

__all__ = ["PAIRED_STAMP", "gemv_paired", "repack_paired", "unpack_paired"]

PAIRED_STAMP = 25


def _ext():
    from . import _ext as ext

    return ext()


def repack_paired(packed: torch.Tensor) -> torch.Tensor:
    """int32 [M, K/8] in the API format -> the same shape in the paired layout."""
    return _ext().repack_paired(packed)


def unpack_paired(paired: torch.Tensor) -> torch.Tensor:
    """Inverse of repack_paired, bit for bit."""
    return _ext().unpack_paired(paired)


def gemv_paired(paired: torch.Tensor, scales: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """y[B, M] = W x for paired-layout weights (x [B, K] or [K], fp16)."""
    squeeze = x.dim() == 1
    y = _ext().w4a16_gemv_paired(paired, scales, x.unsqueeze(0) if squeeze else x)
    return y[0] if squeeze else y
