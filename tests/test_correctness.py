"""GPU correctness gate: every kernel variant vs the pinned CPU oracle.

Restates tests/test_correctness.py of the reference (the 1e-2 max-abs gate
against an fp32 dequantize-then-matmul of the same packed weights, the
cross-variant checks and the dispatch stamps), with the oracle under oracle/
as the reference and the weights quantized on the GPU by this package, which
is also required to be bit-exact with the oracle's quantizer.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import oracle

pytestmark = pytest.mark.gpu

SHAPES = [(256, 256), (4096, 4096)]
if os.environ.get("DK_FULL_SHAPES") == "1":
    SHAPES += [(4096, 11008), (4096, 14336)]
VERSIONS = [0, 1, 2, 3, 4, 5]
MAX_ABS = 1e-2  # the reference's gate (tests/test_correctness.py:29)
N_RANDOM = int(os.environ.get("DK_N_RANDOM", "3"))
if os.environ.get("DK_FULL_TEST") == "1":
    N_RANDOM = 100


def _ext():
    from decode_kernel import _cuda  # a missing extension on a GPU box is a failure

    return _cuda


def _oracle_y(x: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor) -> np.ndarray:
    return oracle.linear_f64(x.cpu().numpy(), packed.cpu().numpy(), scales.cpu().numpy())


def _cross_tol(a: torch.Tensor, b: torch.Tensor, base: float) -> torch.Tensor:
    """`base` plus one fp16 ulp of the larger magnitude: two fp32 summation
    orders can round the same real value to adjacent fp16 outputs."""
    mag = torch.maximum(a.float().abs(), b.float().abs()).cpu().numpy()
    return torch.from_numpy(base + oracle.fp16_ulp(mag))


def _run(m, k, batch, version, seed, reuse=False):
    from decode_kernel import gemv
    from decode_kernel.quantize import quantize_and_pack

    _ext()
    torch.manual_seed(seed)
    w = torch.randn(m, k, device="cuda") * 0.05
    x = torch.randn(batch, k, device="cuda", dtype=torch.float16)
    packed, scales = quantize_and_pack(w)
    p_ref, s_ref = oracle.quantize_and_pack(w.cpu().numpy())
    assert np.array_equal(packed.cpu().numpy(), p_ref), "GPU quantizer differs from oracle"
    assert np.array_equal(scales.cpu().numpy().view(np.uint16), s_ref.view(np.uint16))
    y = gemv(packed, scales, x, version=version, split_k=4 if version == 4 else 1,
             reuse_weights=reuse)
    torch.cuda.synchronize()
    assert y.shape == (batch, m) and y.dtype == torch.float16
    err = oracle.max_abs_err(y.cpu().numpy(), _oracle_y(x, packed, scales))
    assert err < MAX_ABS, (
        f"max abs err {err:.4e} >= {MAX_ABS} for v{version} M={m} K={k} B={batch} "
        f"seed={seed} reuse={reuse}"
    )
    return err


@pytest.mark.parametrize("version", VERSIONS)
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("batch", [1, 4])
def test_versions_against_fp32_reference(version, shape, batch):
    m, k = shape
    for i in range(N_RANDOM):
        _run(m, k, batch, version, seed=1000 + i)


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("batch", [1, 4, 16])
def test_reuse_against_fp32_reference(shape, batch):
    m, k = shape
    for i in range(N_RANDOM):
        _run(m, k, batch, 5, seed=2000 + i, reuse=True)


def test_reuse_weights_matches_streaming():
    # tests/test_correctness.py:77-89 (1e-3, widened by one fp16 ulp of |y|).
    from decode_kernel import gemv
    from decode_kernel.quantize import quantize_and_pack

    _ext()
    torch.manual_seed(1)
    m, k, b = 256, 512, 8
    w = torch.randn(m, k, device="cuda") * 0.05
    x = torch.randn(b, k, device="cuda", dtype=torch.float16)
    packed, scales = quantize_and_pack(w)
    y_stream = gemv(packed, scales, x, version=5, reuse_weights=False)
    y_reuse = gemv(packed, scales, x, version=5, reuse_weights=True)
    diff = (y_stream.float() - y_reuse.float()).abs().cpu()
    assert torch.all(diff <= _cross_tol(y_stream, y_reuse, 1e-3)), float(diff.max())


def test_splitk_matches_v3():
    # tests/test_correctness.py:92-104.
    from decode_kernel import gemv
    from decode_kernel.quantize import quantize_and_pack

    _ext()
    torch.manual_seed(2)
    m, k = 256, 1024
    w = torch.randn(m, k, device="cuda") * 0.05
    x = torch.randn(1, k, device="cuda", dtype=torch.float16)
    packed, scales = quantize_and_pack(w)
    y3 = gemv(packed, scales, x, version=3)
    y4 = gemv(packed, scales, x, version=4, split_k=4)
    diff = (y3.float() - y4.float()).abs().cpu()
    assert torch.all(diff <= _cross_tol(y3, y4, 1e-3)), float(diff.max())


def test_kernel_stamps_are_distinct():
    # tests/test_correctness.py:107-121 and bench/stamp_check.py:56-66.
    from decode_kernel import gemv
    from decode_kernel.quantize import quantize_and_pack

    ext = _ext()
    torch.manual_seed(4)
    m, k = 256, 512
    w = torch.randn(m, k, device="cuda") * 0.05
    x = torch.randn(1, k, device="cuda", dtype=torch.float16)
    packed, scales = quantize_and_pack(w)
    seen = {}
    for v in range(6):
        gemv(packed, scales, x, version=v, split_k=4 if v == 4 else 1)
        seen[v] = int(ext.last_kernel_stamp())
    assert seen == {0: 0, 1: 1, 2: 2, 3: 3, 4: 4, 5: 5}, seen
    gemv(packed, scales, x, version=5, reuse_weights=True)
    assert int(ext.last_kernel_stamp()) == 15
    assert int(ext.last_kernel_stamp()) == -1  # read-and-clear


def test_stamp_recorded_only_for_launches():
    """The host records the stamp when a launch succeeds: a describe call, a
    rejected call and a call with nothing to do leave it unset, and the
    stamp is per device (read on the current one)."""
    import ctypes

    from decode_kernel import _abi
    from decode_kernel.quantize import quantize_and_pack

    ext = _ext()
    lib = _abi.load()
    m, k = 512, 1024
    packed, scales = quantize_and_pack(torch.randn(m, k, device="cuda") * 0.05)
    x = torch.randn(1, k, device="cuda", dtype=torch.float16)
    y = torch.empty(1, m, device="cuda", dtype=torch.float16)
    cfg = _abi.default_config(lib)
    stream = torch.cuda.current_stream().cuda_stream
    ext.last_kernel_stamp()
    assert _abi.describe(lib, m, k, 1)["launches"] == 1
    assert int(ext.last_kernel_stamp()) == -1
    # K not a multiple of the group size: rejected before any launch.
    rc = lib.dk_w4a16_gemv(packed.data_ptr(), scales.data_ptr(), x.data_ptr(), y.data_ptr(), m,
                           k - 64, 1, ctypes.byref(cfg), None, 0, stream)
    assert rc != _abi.DK_OK
    assert int(ext.last_kernel_stamp()) == -1
    # B = 0: nothing to launch.
    rc = lib.dk_w4a16_gemv(packed.data_ptr(), scales.data_ptr(), x.data_ptr(), y.data_ptr(), m, k,
                           0, ctypes.byref(cfg), None, 0, stream)
    assert rc == _abi.DK_OK
    assert int(ext.last_kernel_stamp()) == -1
    rc = lib.dk_w4a16_gemv(packed.data_ptr(), scales.data_ptr(), x.data_ptr(), y.data_ptr(), m, k,
                           1, ctypes.byref(cfg), None, 0, stream)
    assert rc == _abi.DK_OK
    assert int(ext.last_kernel_stamp()) == 5
    assert int(ext.last_kernel_stamp()) == -1


def test_v1_multiwarp_matches_v1():
    # tests/test_correctness.py:124-142, plus every waves-per-row value.
    from decode_kernel import gemv
    from decode_kernel.quantize import quantize_and_pack

    ext = _ext()
    torch.manual_seed(3)
    m, k = 256, 1024
    w = torch.randn(m, k, device="cuda") * 0.05
    x = torch.randn(1, k, device="cuda", dtype=torch.float16)
    packed, scales = quantize_and_pack(w)
    y1 = gemv(packed, scales, x, version=1, warps_per_row=1)
    assert int(ext.last_kernel_stamp()) == 1
    for wpr in range(2, 9):
        yw = gemv(packed, scales, x, version=1, warps_per_row=wpr)
        assert int(ext.last_kernel_stamp()) == 10 + wpr
        assert (y1.float() - yw.float()).abs().max().item() < 1e-2
