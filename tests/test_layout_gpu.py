"""The kernel-native paired weight layout on the GPU.

* dk_repack_paired / dk_unpack_paired against the oracle's numpy permutation
  (bit for bit) on random words, including every nibble value, and the round
  trip unpack(repack(w)) == w at every benchmark shape.
* The v5 GEMV on paired weights (stamp 25) against the oracle's float64
  product of the original weights with the tight bound used for every
  product path (half an fp16 ulp of |y| + 1e-3), one-hot exactness, its
  agreement with the logical-layout GEMV, and the ctypes entry point.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle

pytestmark = pytest.mark.gpu

SHAPES = [(4096, 4096), (11008, 4096), (4096, 11008), (28672, 8192), (8192, 28672)]


def _check_tight(y: torch.Tensor, y_ref: np.ndarray, label: str):
    err = np.abs(y.float().cpu().numpy().astype(np.float64) - y_ref)
    assert err.max() < 1e-2, f"{label}: max abs err {err.max():.3e}"
    tight = 0.5 * oracle.fp16_ulp(y_ref) + 1e-3
    bad = np.argwhere(err > tight)
    assert bad.size == 0, f"{label}: {len(bad)} beyond half-ulp+1e-3, first {bad[:3].tolist()}"


def test_repack_matches_oracle_on_random_words():
    from decode_kernel import repack_paired, unpack_paired

    rng = np.random.Generator(np.random.PCG64(1))
    w = rng.integers(0, 1 << 32, size=(333, 64), dtype=np.uint64).astype(np.uint32).view(np.int32)
    wd = torch.from_numpy(w).cuda()
    p = repack_paired(wd)
    np.testing.assert_array_equal(p.cpu().numpy(), oracle.repack_paired(w))
    assert torch.equal(unpack_paired(p), wd)
    # Hand-permuted words from the oracle's known answers.
    kat = torch.tensor(np.array([[0x76543210, 0x09ABCDEF] + [0] * 14], dtype=np.uint32).view(np.int32)).cuda()
    got = repack_paired(kat).cpu().numpy().view(np.uint32)[0]
    assert int(got[0]) == 0x75316420 and int(got[1]) == 0x0ACE9BDF


@pytest.mark.parametrize("m,k", SHAPES)
def test_round_trip_and_gemv_at_full_size(m, k):
    from decode_kernel import _cuda, gemv, gemv_paired, quantize_and_pack, repack_paired, unpack_paired

    gen = torch.Generator(device="cuda").manual_seed(m + k)
    packed, scales = quantize_and_pack(torch.randn(m, k, device="cuda", generator=gen) * 0.02)
    paired = repack_paired(packed)
    assert torch.equal(unpack_paired(paired), packed)
    x = torch.randn(1, k, device="cuda", generator=gen).half()
    y = gemv_paired(paired, scales, x)
    assert int(_cuda.last_kernel_stamp()) == 25
    _check_tight(y, oracle.linear_f64(x.cpu().numpy(), packed.cpu().numpy(), scales.cpu().numpy()),
                 f"paired {m}x{k}")
    # Same products as the logical layout, summed in another pair order.
    y_logical = gemv(packed, scales, x)
    tol = 1e-3 + torch.from_numpy(oracle.fp16_ulp(y_logical.float().cpu().numpy())).cuda()
    assert bool(((y.float() - y_logical.float()).abs() <= tol).all())


@pytest.mark.parametrize("m,k,b", [(1, 128, 1), (17, 384, 2), (4097, 256, 3), (512, 1024, 4),
                                   (256, 4096, 7), (4096, 4096, 16)])
def test_gemv_paired_edge_shapes_and_batches(m, k, b):
    from decode_kernel import gemv_paired, repack_paired

    w, x = oracle.make_case(m, k, b, seed=m + k + b, w_std=0.05)
    packed, scales = oracle.quantize_and_pack(w)
    paired = repack_paired(torch.from_numpy(packed).cuda())
    y = gemv_paired(paired, torch.from_numpy(scales).cuda(), torch.from_numpy(x).cuda())
    _check_tight(y, oracle.linear_f64(x, packed, scales), f"paired {m}x{k} B={b}")


def test_one_hot_is_exact_and_vector_input():
    from decode_kernel import gemv_paired, repack_paired

    w, _ = oracle.make_case(300, 512, 1, seed=3, w_std=0.5)
    packed, scales = oracle.quantize_and_pack(w)
    paired = repack_paired(torch.from_numpy(packed).cuda())
    sd = torch.from_numpy(scales).cuda()
    wq = oracle.dequantize(packed, scales, dtype=np.float64)
    for k in (0, 1, 7, 8, 130, 511):
        x = torch.zeros(512, device="cuda", dtype=torch.float16)
        x[k] = 1.0
        y = gemv_paired(paired, sd, x)
        assert y.shape == (300,)
        np.testing.assert_array_equal(y.cpu().numpy(), wq[:, k].astype(np.float16))


def test_c_abi_paired_matches_extension():
    from decode_kernel import _abi, gemv_paired, repack_paired

    lib = _abi.load()
    w, x = oracle.make_case(1000, 2048, 3, seed=8)
    packed, scales = oracle.quantize_and_pack(w)
    pd = torch.from_numpy(packed).cuda()
    sd = torch.from_numpy(scales).cuda()
    xd = torch.from_numpy(x).cuda()
    stream = torch.cuda.current_stream().cuda_stream
    paired = torch.empty_like(pd)
    _abi.check(lib, lib.dk_repack_paired(pd.data_ptr(), paired.data_ptr(), 1000, 2048, stream))
    assert torch.equal(paired, repack_paired(pd))
    y = torch.empty(3, 1000, dtype=torch.float16, device="cuda")
    _abi.check(lib, lib.dk_w4a16_gemv_paired(paired.data_ptr(), sd.data_ptr(), xd.data_ptr(),
                                             y.data_ptr(), 1000, 2048, 3, stream))
    assert torch.equal(y, gemv_paired(paired, sd, xd))
    back = torch.empty_like(pd)
    _abi.check(lib, lib.dk_unpack_paired(paired.data_ptr(), back.data_ptr(), 1000, 2048, stream))
    assert torch.equal(back, pd)


def test_rejected_inputs():
    from decode_kernel import gemv_paired, repack_paired

    with pytest.raises(RuntimeError, match="group size"):
        repack_paired(torch.zeros(4, 25, dtype=torch.int32, device="cuda"))
    with pytest.raises(RuntimeError, match="int32"):
        repack_paired(torch.zeros(4, 16, dtype=torch.float32, device="cuda"))
    with pytest.raises(RuntimeError, match="x.shape"):
        gemv_paired(torch.zeros(4, 16, dtype=torch.int32, device="cuda"),
                    torch.zeros(4, 1, dtype=torch.float16, device="cuda"),
                    torch.zeros(1, 256, dtype=torch.float16, device="cuda"))
