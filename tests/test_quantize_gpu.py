"""The HIP quantizer (dk_quantize_pack_f32 / _cuda.quantize_and_pack) against
the oracle, bit for bit.

The reference quantizer is python/decode_kernel/quantize.py:26-51; the oracle
restates it in numpy float32 and is pinned by tests/test_oracle.py. Here:

* the reference's known answer and hand-derived words (ties to even, scale
  floor, ±7 saturation) through the GPU;
* seeded random matrices of several distributions against the oracle;
* every benchmark shape at full size against the torch formulation on the
  same GPU (a second, independent code path), a random sample of rows
  against the oracle, and the exact round trip
  quantize(dequantize(quantize(W))) == quantize(W);
* edge shapes (one group, M = 1, M = 0, K = 0), non-fp32 and
  non-contiguous inputs, rejected shapes, and the ctypes C ABI.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle

pytestmark = pytest.mark.gpu

FULL_SHAPES = {
    "c0": (4096, 4096),
    "c1": (11008, 4096),
    "c2": (4096, 11008),
    "c4a": (28672, 8192),
    "c4b": (8192, 28672),
}


def _gpu_quantize(w: np.ndarray):
    from decode_kernel import _cuda

    packed, scales = _cuda.quantize_and_pack(torch.from_numpy(w).cuda())
    torch.cuda.synchronize()
    return packed.cpu().numpy(), scales.cpu().numpy()


def _assert_same(got, want, label):
    gp, gs = got
    wp, ws = want
    assert gp.dtype == np.int32 and gs.dtype == np.float16, label
    assert gp.shape == wp.shape and gs.shape == ws.shape, label
    bad = np.argwhere(gp != wp)
    assert bad.size == 0, f"{label}: {len(bad)} packed words differ, first {bad[:3].tolist()}"
    bad = np.argwhere(gs.view(np.uint16) != ws.view(np.uint16))
    assert bad.size == 0, f"{label}: {len(bad)} scales differ, first {bad[:3].tolist()}"


# ----------------------------------------------------------- known answers ---
def test_reference_kat_through_gpu():
    # tests/test_quantize.py:41-53 of the reference.
    w = np.zeros((1, 128), np.float32)
    w[0, 0], w[0, 1] = 7.0, -7.0
    p, s = _gpu_quantize(w)
    assert int(p[0, 0]) & 0xFFFFFFFF == 0x00000097
    assert (p[0, 1:] == 0).all()
    assert s.view(np.uint16)[0, 0] == 0x3C00


def test_ties_round_half_even():
    # amax 7 -> scale exactly 1; amax 1.75 -> scale exactly 0.25.
    halves = np.array([0.5, 1.5, 2.5, 3.5, 4.5, 5.5, 6.5], np.float32)
    expect = np.array([0, 2, 2, 4, 4, 6, 6])
    for scale in (1.0, 0.25):
        w = np.zeros((2, 128), np.float32)
        w[:, 127] = 7 * scale
        w[0, :7] = halves * scale
        w[1, :7] = -halves * scale
        got = _gpu_quantize(w)
        q = oracle.unpack_to_int(got[0])
        assert (q[0, :7] == expect).all(), (scale, q[0, :7])
        assert (q[1, :7] == -expect).all(), (scale, q[1, :7])
        assert q[0, 127] == 7
        _assert_same(got, oracle.quantize_and_pack(w), f"ties scale {scale}")


def test_scale_floor_and_zero_groups():
    # A zero group: scale clamps to fp32(1e-8), which rounds to fp16 0; all q 0.
    # A tiny group (amax 3.5e-8 < 7e-8): the floor 1e-8 is the scale, and
    # fp32(3.5e-8) / fp32(1e-8) is exactly 3.5, a tie that rounds to 4.
    w = np.zeros((3, 256), np.float32)
    w[1, 0], w[1, 1], w[1, 2] = 3.5e-8, -2e-8, 1e-9
    w[2, 128:] = np.linspace(-1e-7, 1e-7, 128, dtype=np.float32)
    got = _gpu_quantize(w)
    _assert_same(got, oracle.quantize_and_pack(w), "floor")
    assert (got[0][0] == 0).all()
    assert (got[1].view(np.uint16)[0] == 0).all()
    q = oracle.unpack_to_int(got[0])
    assert q[1, 0] == 4 and q[1, 1] == -2 and q[1, 2] == 0
    assert q[2, 128] == -7 and q[2, 255] == 7


@pytest.mark.parametrize("m,k,seed,std", [
    (1, 128, 0, 1.0),
    (3, 384, 1, 0.02),
    (37, 1280, 2, 0.05),
    (256, 4096, 3, 0.02),
    (129, 11008, 4, 3.0),
    (64, 28672, 5, 1e3),
])
def test_random_matches_oracle(m, k, seed, std):
    rng = np.random.Generator(np.random.PCG64(seed))
    w = (rng.standard_normal((m, k)) * std).astype(np.float32)
    _assert_same(_gpu_quantize(w), oracle.quantize_and_pack(w), f"{m}x{k} std {std}")


def test_mixed_magnitude_groups_and_outliers():
    rng = np.random.Generator(np.random.PCG64(7))
    w = rng.standard_normal((96, 1024)).astype(np.float32)
    w *= np.float32(10.0) ** rng.integers(-9, 4, size=(96, 8, 1)).repeat(128, axis=2).reshape(96, 1024)
    w[::5, ::97] *= np.float32(50.0)  # one outlier per group on some rows
    _assert_same(_gpu_quantize(w), oracle.quantize_and_pack(w), "mixed magnitudes")


def test_values_on_exact_steps():
    # Every w an integer multiple of an exact power-of-two scale: q must equal
    # the multiplier, unrounded.
    rng = np.random.Generator(np.random.PCG64(11))
    mult = rng.integers(-7, 8, size=(64, 512)).astype(np.float32)
    mult[:, ::128] = 7.0  # amax = 7 * scale in every group
    scale = np.float32(2.0) ** rng.integers(-12, 3, size=(64, 4, 1)).astype(np.float32)
    w = (mult.reshape(64, 4, 128) * scale).reshape(64, 512).astype(np.float32)
    p, s = _gpu_quantize(w)
    assert (oracle.unpack_to_int(p) == mult).all()
    assert (s.astype(np.float32) == scale[..., 0]).all()


# -------------------------------------------------------------- full sizes ---
@pytest.mark.parametrize("name", list(FULL_SHAPES))
def test_full_size_against_torch_formulation_and_oracle_rows(name):
    from decode_kernel import _cuda
    from decode_kernel.quantize import dequantize, quantize_and_pack_torch

    m, k = FULL_SHAPES[name]
    gen = torch.Generator(device="cuda").manual_seed(1000 + m + k)
    w = torch.randn(m, k, device="cuda", generator=gen) * 0.02
    packed, scales = _cuda.quantize_and_pack(w)
    tp, ts = quantize_and_pack_torch(w)
    assert torch.equal(packed, tp), f"{name}: packed differs from the torch formulation"
    assert torch.equal(scales.view(torch.int16), ts.view(torch.int16)), f"{name}: scales differ"

    rows = torch.randperm(m, generator=torch.Generator().manual_seed(m))[:128].sort().values
    w_rows = w[rows.cuda()].cpu().numpy()
    _assert_same((packed[rows.cuda()].cpu().numpy(), scales[rows.cuda()].cpu().numpy()),
                 oracle.quantize_and_pack(w_rows), f"{name} sampled rows")

    # Requantizing the dequantized weights reproduces the same bits (the amax
    # of each group is 7 * its fp16 scale, so every division is exact).
    p2, s2 = _cuda.quantize_and_pack(dequantize(packed, scales))
    assert torch.equal(p2, packed) and torch.equal(s2.view(torch.int16), scales.view(torch.int16))


def test_gemv_on_gpu_quantized_weights_matches_oracle():
    from decode_kernel import _cuda, gemv

    rng = np.random.Generator(np.random.PCG64(21))
    w = (rng.standard_normal((1024, 2048)) * 0.05).astype(np.float32)
    x = rng.standard_normal((4, 2048)).astype(np.float16)
    packed, scales = _cuda.quantize_and_pack(torch.from_numpy(w).cuda())
    y = gemv(packed, scales, torch.from_numpy(x).cuda())
    op, os_ = oracle.quantize_and_pack(w)
    err = oracle.max_abs_err(y.float().cpu().numpy(), oracle.linear_f64(x, op, os_))
    assert err < 1e-2


# ------------------------------------------------------- shapes and inputs ---
def test_edge_shapes_and_dtypes():
    from decode_kernel import _cuda, quantize_and_pack

    p, s = _cuda.quantize_and_pack(torch.zeros(0, 256, device="cuda"))
    assert p.shape == (0, 32) and s.shape == (0, 2)
    p, s = _cuda.quantize_and_pack(torch.zeros(5, 0, device="cuda"))
    assert p.shape == (5, 0) and s.shape == (5, 0)

    rng = np.random.Generator(np.random.PCG64(3))
    w = rng.standard_normal((128, 640)).astype(np.float32)
    want = oracle.quantize_and_pack(w)
    wt = torch.from_numpy(w).cuda()
    # Non-contiguous (a transposed copy viewed back) and the package API.
    nc = wt.t().contiguous().t()
    assert not nc.is_contiguous()
    _assert_same(tuple(t.cpu().numpy() for t in quantize_and_pack(nc)), want, "non-contiguous")
    # fp16 input: quantized as its fp32 value.
    wh = wt.half()
    _assert_same(tuple(t.cpu().numpy() for t in quantize_and_pack(wh)),
                 oracle.quantize_and_pack(wh.float().cpu().numpy()), "fp16 input")


def test_rejected_inputs():
    from decode_kernel import _cuda, quantize_and_pack

    with pytest.raises(RuntimeError, match="group_size"):
        _cuda.quantize_and_pack(torch.zeros(4, 200, device="cuda"))
    with pytest.raises(RuntimeError, match="fp32"):
        _cuda.quantize_and_pack(torch.zeros(4, 128, device="cuda", dtype=torch.float16))
    with pytest.raises(RuntimeError, match="CUDA"):
        _cuda.quantize_and_pack(torch.zeros(4, 128))
    with pytest.raises(ValueError, match="group_size"):
        quantize_and_pack(torch.zeros(4, 200, device="cuda"))


def test_c_abi_direct_matches_extension():
    from decode_kernel import _abi, _cuda

    lib = _abi.load()
    rng = np.random.Generator(np.random.PCG64(5))
    w = torch.from_numpy(rng.standard_normal((300, 1536)).astype(np.float32)).cuda()
    p = torch.empty(300, 192, dtype=torch.int32, device="cuda")
    s = torch.empty(300, 12, dtype=torch.float16, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    _abi.check(lib, lib.dk_quantize_pack_f32(w.data_ptr(), 300, 1536, p.data_ptr(), s.data_ptr(),
                                             stream))
    ep, es = _cuda.quantize_and_pack(w)
    assert torch.equal(p, ep) and torch.equal(s.view(torch.int16), es.view(torch.int16))
    # Misaligned fp32 input is refused before any launch.
    rc = lib.dk_quantize_pack_f32(w.data_ptr() + 4, 1, 128, p.data_ptr(), s.data_ptr(), stream)
    assert rc == _abi.DK_ERR_INVALID_ARGUMENT
    assert b"aligned" in lib.dk_last_error()
