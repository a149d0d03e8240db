"""CPU tests for the product packing format (decode_kernel.quantize).

The first four tests restate the reference's packing gate
(tests/test_quantize.py:16-61) against this package; the rest require
bit-exact agreement with the pinned oracle on the same inputs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from decode_kernel.quantize import GROUP_SIZE, dequantize, quantize_and_pack, unpack_to_int
from oracle import oracle


@pytest.mark.parametrize("shape", [(8, 128), (16, 256), (32, 512)])
def test_pack_unpack_q_roundtrip(shape):
    torch.manual_seed(0)
    w = torch.randn(*shape)
    packed, scales = quantize_and_pack(w)
    q = unpack_to_int(packed)
    assert int(q.min()) >= -7 and int(q.max()) <= 7
    recon = dequantize(packed, scales)
    scale = scales.float().repeat_interleave(GROUP_SIZE, dim=1)
    assert torch.allclose(recon, q.float() * scale, atol=1e-6)


@pytest.mark.parametrize("shape", [(8, 128), (16, 256)])
def test_reconstruction_within_half_step(shape):
    torch.manual_seed(0)
    w = torch.randn(*shape)
    packed, scales = quantize_and_pack(w)
    recon = dequantize(packed, scales)
    scale = scales.float().repeat_interleave(GROUP_SIZE, dim=1)
    err = (recon - w.float()).abs()
    assert torch.all(err <= 0.5 * scale + 1e-3)


def test_pack_layout_low_nibble_first():
    w = torch.zeros(1, 128)
    w[0, 0] = 7.0
    w[0, 1] = -7.0
    packed, scales = quantize_and_pack(w)
    word = int(packed[0, 0].item()) & 0xFFFFFFFF
    assert word & 0xF == 7
    assert (word >> 4) & 0xF == 9
    assert scales.shape == (1, 1)
    assert abs(float(scales[0, 0]) - 1.0) < 1e-3


def test_zero_group_does_not_nan():
    w = torch.zeros(2, 128)
    packed, scales = quantize_and_pack(w)
    recon = dequantize(packed, scales)
    assert torch.isfinite(recon).all()
    assert torch.isfinite(scales.float()).all()


def test_rejects_bad_shapes():
    with pytest.raises(ValueError):
        quantize_and_pack(torch.zeros(128))
    with pytest.raises(ValueError):
        quantize_and_pack(torch.zeros(2, 100))


@pytest.mark.parametrize(
    "m,k,seed,std",
    [(8, 128, 0, 1.0), (37, 256, 1, 0.02), (64, 4096, 2, 0.05), (24, 11008, 3, 0.02), (5, 384, 4, 3.0)],
)
def test_bit_exact_with_oracle(m, k, seed, std):
    w, _ = oracle.make_case(m, k, 1, seed, std)
    p_ref, s_ref = oracle.quantize_and_pack(w)
    packed, scales = quantize_and_pack(torch.from_numpy(w))
    assert packed.dtype == torch.int32 and scales.dtype == torch.float16
    assert np.array_equal(packed.numpy(), p_ref)
    assert np.array_equal(scales.numpy().view(np.uint16), s_ref.view(np.uint16))
    assert np.array_equal(unpack_to_int(packed).numpy(), oracle.unpack_to_int(p_ref))
    assert np.array_equal(dequantize(packed, scales).numpy(), oracle.dequantize(p_ref, s_ref))


def test_torch_randn_inputs_match_oracle():
    # The reference tests draw weights with torch.manual_seed + randn.
    for shape in [(8, 128), (16, 256), (32, 512)]:
        torch.manual_seed(0)
        w = torch.randn(*shape) * 0.05
        packed, scales = quantize_and_pack(w)
        p_ref, s_ref = oracle.quantize_and_pack(w.numpy())
        assert np.array_equal(packed.numpy(), p_ref)
        assert np.array_equal(scales.numpy().view(np.uint16), s_ref.view(np.uint16))


def test_unpack_handles_minus_eight():
    packed = torch.tensor([[0x88888888 - (1 << 32)] * 16], dtype=torch.int32)
    assert unpack_to_int(packed).unique().tolist() == [-8]


def test_product_reference_helper_matches_oracle():
    from decode_kernel.reference import linear_fp32, max_abs_err

    w, x = oracle.make_case(48, 512, 3, 9, 0.05)
    p, s = oracle.quantize_and_pack(w)
    y = linear_fp32(torch.from_numpy(x), torch.from_numpy(p), torch.from_numpy(s))
    assert max_abs_err(y, torch.from_numpy(oracle.linear_f64(x, p, s))) < 1e-4
