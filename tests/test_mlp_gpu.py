"""The fused MLP decode step (dk_gate_up_silu, dk_mlp_decode) against the oracle.

h = fp16(silu(Wg x) * (Wu x)) is checked against the float64 composition in
oracle.gate_up_silu_f64 within half an fp16 ulp of |h| + 1e-3 (the one fp16
rounding plus fp32 accumulation of g and u); y = Wd h is checked against
oracle.linear_f64 of the kernel's own h with the GEMV's bound, and end to end
against oracle.mlp_decode_f64 with the reference's 1e-2 gate. Shapes: the
Llama-7B MLP (I = 11008, H = 4096), the per-GPU Llama-70B shard at TP = 8
(I = 3584, H = 8192), the full Llama-70B MLP (I = 28672, H = 8192, every
row, in row blocks), ragged shapes in every dispatch range, batches 1-33,
and empty dimensions.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle

pytestmark = pytest.mark.gpu

MAX_ABS = 1e-2


def _weights(i: int, h: int, seed: int, std: float = 0.02):
    """Quantized gate/up [I, H] and down [H, I] on the GPU (device quantizer,
    bit-exact with the oracle's) plus their numpy copies. Down is None when
    I is not a multiple of the group size (gate/up-only cases)."""
    from decode_kernel import quantize_and_pack

    gen = torch.Generator(device="cuda").manual_seed(seed)
    out = []
    shapes = ((i, h), (i, h)) + (((h, i),) if i % 128 == 0 else ())
    for shape in shapes:
        p, s = quantize_and_pack(torch.randn(*shape, device="cuda", generator=gen) * std)
        out += [p, s]
    if len(out) == 4:
        out += [None, None]
    return out, [None if t is None else t.cpu().numpy() for t in out]


def _x(b: int, h: int, seed: int) -> torch.Tensor:
    gen = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn(b, h, device="cuda", generator=gen).half()


def _check_tight(got: np.ndarray, ref: np.ndarray, label: str):
    err = np.abs(got.astype(np.float64) - ref)
    assert err.max() < MAX_ABS, f"{label}: max abs err {err.max():.3e}"
    tight = 0.5 * oracle.fp16_ulp(ref) + 1e-3
    bad = np.argwhere(err > tight)
    assert bad.size == 0, f"{label}: {len(bad)} outputs beyond half-ulp+1e-3, first {bad[:3].tolist()}"


@pytest.mark.parametrize("i,h,b", [
    (256, 128, 1), (256, 128, 3), (384, 640, 2), (1000, 256, 5), (11008, 4096, 1),
    (11008, 4096, 4), (3584, 8192, 1), (3584, 8192, 2), (11008, 4096, 8), (3584, 8192, 16),
    (11008, 4096, 16), (11008, 2048, 16), (3584, 8192, 33), (5000, 4224, 20),
])
def test_mlp_step_matches_oracle(i, h, b):
    from decode_kernel import _cuda, gate_up_silu, mlp_decode

    if i % 128:  # gate/up only: I need not be a multiple of 128 there
        (gp, gs, up, us, _, _), (ngp, ngs, nup, nus, _, _) = _weights(i, h, seed=i + h)
        x = _x(b, h, seed=b)
        hk = gate_up_silu(x, gp, gs, up, us)
        assert int(_cuda.last_kernel_stamp()) == 20
        _check_tight(hk.float().cpu().numpy(),
                     oracle.gate_up_silu_f64(x.cpu().numpy(), ngp, ngs, nup, nus), f"h {i}x{h}")
        return
    (gp, gs, up, us, dp, ds), (ngp, ngs, nup, nus, ndp, nds) = _weights(i, h, seed=i + h)
    x = _x(b, h, seed=b)
    xn = x.cpu().numpy()
    hk = gate_up_silu(x, gp, gs, up, us)
    assert int(_cuda.last_kernel_stamp()) == 20
    h_ref = oracle.gate_up_silu_f64(xn, ngp, ngs, nup, nus)
    hkn = hk.cpu().numpy()
    _check_tight(hkn.astype(np.float64), h_ref, f"h {i}x{h} B={b}")
    y = mlp_decode(x, gp, gs, up, us, dp, ds)
    # The down projection is the GEMV on h: v5 for one row, the reuse path
    # for a batch.
    assert int(_cuda.last_kernel_stamp()) == (15 if b > 1 else 5)
    yn = y.float().cpu().numpy()
    _check_tight(yn, oracle.linear_f64(hkn, ndp, nds), f"y from kernel h {i}x{h} B={b}")
    y_ref = oracle.mlp_decode_f64(xn, ngp, ngs, nup, nus, ndp, nds)
    assert oracle.max_abs_err(yn, y_ref) < MAX_ABS
    # The fused step is exactly gate_up_silu followed by gemv on its output.
    from decode_kernel import gemv

    assert torch.equal(y, gemv(dp, ds, hk, reuse_weights=b > 1))


# Ragged shapes in every I range (<= 2048, 4096, above) and H range (<= 4096,
# 8192, above) the gate/up dispatch tells apart.
GATE_UP_SHAPES = [(1000, 4224), (2000, 8320), (3000, 4224), (3000, 8320), (5000, 4224),
                  (4500, 8320), (1800, 6144), (700, 3968), (5000, 5120), (2752, 4096),
                  (3000, 6144), (1000, 4096), (600, 8192), (1376, 8192)]


@pytest.mark.parametrize("i,h", GATE_UP_SHAPES)
def test_gate_up_every_dispatch_class(i, h):
    # Batches 1-8 cover every streaming tile size (one row, and tiles of 2, 3
    # and 4 rows, the last one partly empty at B = 5 and 7); from 3 rows at
    # I > 2048, and from 9 rows at I > 1024, the MFMA tiles run instead (with
    # both operands staged in LDS from 8 rows, double buffered at 9-16 rows
    # up to I = 4096 where the scales pair: I = 1800, 2752 and 3000, and
    # below 9 rows with four x loads per block at I = 2752 and 3000). Where
    # the scales pair at 513-2048 rows the double-buffered tiles run once
    # B I > 8192: I = 1800 from 5 rows, I = 1376 from 6, I = 1000 from 9,
    # I = 600 at 16. Each output row depends on its own activation row only,
    # so the first b rows of one 16-row case give the reference for every b.
    from decode_kernel import _cuda, gate_up_silu

    (gp, gs, up, us, _, _), (ngp, ngs, nup, nus, _, _) = _weights(i, h, seed=i + h)
    x16 = _x(16, h, seed=i)
    h_ref = oracle.gate_up_silu_f64(x16.cpu().numpy(), ngp, ngs, nup, nus)
    for b in (1, 2, 3, 4, 5, 6, 7, 8, 12, 16):
        hk = gate_up_silu(x16[:b].contiguous(), gp, gs, up, us)
        assert int(_cuda.last_kernel_stamp()) == 20
        _check_tight(hk.float().cpu().numpy(), h_ref[:b], f"h {i}x{h} B={b}")


def test_llama70b_full_mlp_every_row():
    # Every row of h (28672) and of y (8192), against the float64 oracle in
    # blocks of rows (the unpacked weights of the whole matrix in float64
    # would take 1.9 GB each).
    from decode_kernel import gate_up_silu, mlp_decode

    i, h = 28672, 8192
    (gp, gs, up, us, dp, ds), _ = _weights(i, h, seed=70)
    x = _x(1, h, seed=7)
    xn = x.cpu().numpy()
    hk = gate_up_silu(x, gp, gs, up, us)
    y = mlp_decode(x, gp, gs, up, us, dp, ds)
    hkn = hk.float().cpu().numpy()
    for r0 in range(0, i, 4096):
        rows = slice(r0, r0 + 4096)
        h_ref = oracle.gate_up_silu_f64(xn, gp[rows].cpu().numpy(), gs[rows].cpu().numpy(),
                                        up[rows].cpu().numpy(), us[rows].cpu().numpy())
        _check_tight(hkn[:, rows], h_ref, f"h 70B rows {r0}..")
    yn = y.float().cpu().numpy()
    hk_np = hk.cpu().numpy()
    for r0 in range(0, h, 1024):
        rows = slice(r0, r0 + 1024)
        y_ref = oracle.linear_f64(hk_np, dp[rows].cpu().numpy(), ds[rows].cpu().numpy())
        _check_tight(yn[:, rows], y_ref, f"y 70B rows {r0}..")


def test_fused_agrees_with_unfused_composition():
    # Three GEMVs with fp16 g and u, then SiLU*mul in fp32: the composition a
    # caller of the reference would write. It rounds g and u to fp16 first,
    # so it may differ from the fused step by a few fp16 ulps of h.
    from decode_kernel import gemv, mlp_decode

    (gp, gs, up, us, dp, ds), _ = _weights(11008, 4096, seed=3)
    x = _x(2, 4096, seed=3)
    g = gemv(gp, gs, x).float()
    u = gemv(up, us, x).float()
    h_unfused = (torch.nn.functional.silu(g) * u).half()
    from decode_kernel import gate_up_silu

    h = gate_up_silu(x, gp, gs, up, us)
    diff = (h.float() - h_unfused.float()).abs()
    bound = 4 * torch.from_numpy(oracle.fp16_ulp(h.float().cpu().numpy())).cuda() + 1e-3
    assert bool((diff <= bound).all()), float(diff.max())
    y = mlp_decode(x, gp, gs, up, us, dp, ds)
    y_unfused = gemv(dp, ds, h_unfused)
    assert float((y.float() - y_unfused.float()).abs().max()) < MAX_ABS


def test_one_hot_activation_is_exact():
    # x = e_k: g and u are single scaled weights, so h = fp16(silu(wg) * wu)
    # up to the fp32 SiLU (within one fp16 rounding of the float64 value).
    from decode_kernel import gate_up_silu

    (gp, gs, up, us, _, _), (ngp, ngs, nup, nus, _, _) = _weights(512, 1024, seed=11, std=0.5)
    x = torch.zeros(1, 1024, device="cuda", dtype=torch.float16)
    x[0, 700] = 1.0
    h = gate_up_silu(x, gp, gs, up, us).float().cpu().numpy()[0]
    wg = oracle.dequantize(ngp, ngs, dtype=np.float64)[:, 700]
    wu = oracle.dequantize(nup, nus, dtype=np.float64)[:, 700]
    ref = oracle.silu_f64(wg) * wu
    assert np.all(np.abs(h - ref) <= 0.5 * oracle.fp16_ulp(ref) + 1e-6)


def test_empty_and_vector_inputs():
    from decode_kernel import QuantizedMLP, gate_up_silu, mlp_decode

    (gp, gs, up, us, dp, ds), _ = _weights(256, 128, seed=1)
    assert mlp_decode(torch.zeros(0, 128, device="cuda", dtype=torch.float16),
                      gp, gs, up, us, dp, ds).shape == (0, 128)
    x1 = _x(1, 128, seed=4)
    y1 = mlp_decode(x1[0], gp, gs, up, us, dp, ds)
    assert y1.shape == (128,) and torch.equal(y1, mlp_decode(x1, gp, gs, up, us, dp, ds)[0])
    assert gate_up_silu(x1[0], gp, gs, up, us).shape == (256,)
    # I = 0: h is empty and y = Wd h is all zeros.
    e = torch.zeros(0, 16, dtype=torch.int32, device="cuda")
    es = torch.zeros(0, 1, dtype=torch.float16, device="cuda")
    d0 = torch.zeros(128, 0, dtype=torch.int32, device="cuda")
    ds0 = torch.zeros(128, 0, dtype=torch.float16, device="cuda")
    y0 = mlp_decode(x1, e, es, e, es, d0, ds0)
    assert y0.shape == (1, 128) and not bool(y0.any())
    # QuantizedMLP on fp32 weights quantizes on the device and runs the step.
    gen = torch.Generator(device="cuda").manual_seed(5)
    wg, wu = (torch.randn(256, 128, device="cuda", generator=gen) for _ in range(2))
    wd = torch.randn(128, 256, device="cuda", generator=gen)
    mlp = QuantizedMLP.from_float(wg, wu, wd)
    assert (mlp.intermediate_size, mlp.hidden_size) == (256, 128)
    assert torch.equal(mlp(x1), mlp_decode(x1, mlp.gate_packed, mlp.gate_scales, mlp.up_packed,
                                           mlp.up_scales, mlp.down_packed, mlp.down_scales))


def test_rejected_shapes():
    from decode_kernel import mlp_decode

    (gp, gs, up, us, dp, ds), _ = _weights(256, 128, seed=2)
    x = _x(1, 128, seed=2)
    with pytest.raises(RuntimeError, match="same shape"):
        mlp_decode(x, gp, gs, up[:128], us[:128], dp, ds)
    with pytest.raises(RuntimeError, match="down must be"):
        mlp_decode(x, gp, gs, up, us, dp[:64], ds[:64])
    with pytest.raises(RuntimeError, match="x.shape"):
        mlp_decode(_x(1, 256, seed=2), gp, gs, up, us, dp, ds)
    (gp3, gs3, up3, us3, _, _), _ = _weights(200, 128, seed=2)  # I = 200: no down
    with pytest.raises(RuntimeError, match="I must be divisible"):
        mlp_decode(x, gp3, gs3, up3, us3, dp[:, :25].contiguous(), ds[:, :1].contiguous())


def test_c_abi_mlp_matches_extension():
    from decode_kernel import _abi, mlp_decode

    lib = _abi.load()
    i, h, b = 1024, 512, 3
    (gp, gs, up, us, dp, ds), _ = _weights(i, h, seed=9)
    x = _x(b, h, seed=9)
    y = torch.empty(b, h, dtype=torch.float16, device="cuda")
    ws_bytes = lib.dk_mlp_workspace_bytes(i, h, b)
    assert ws_bytes == b * i * 2
    ws = torch.empty(ws_bytes // 2, dtype=torch.float16, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    _abi.check(lib, lib.dk_mlp_decode(gp.data_ptr(), gs.data_ptr(), up.data_ptr(), us.data_ptr(),
                                      dp.data_ptr(), ds.data_ptr(), x.data_ptr(), y.data_ptr(),
                                      i, h, b, ws.data_ptr(), ws_bytes, stream))
    assert torch.equal(y, mlp_decode(x, gp, gs, up, us, dp, ds))
    hk = torch.empty(b, i, dtype=torch.float16, device="cuda")
    _abi.check(lib, lib.dk_gate_up_silu(gp.data_ptr(), gs.data_ptr(), up.data_ptr(), us.data_ptr(),
                                        x.data_ptr(), hk.data_ptr(), i, h, b, stream))
    assert torch.equal(hk, ws.view(b, i))


@pytest.mark.parametrize("i,h,b", [(11008, 4096, 4), (5000, 8192, 8), (11008, 4096, 16),
                                   (3584, 8192, 8), (3584, 8192, 16)])
def test_gate_up_tiles_scale_alignment(i, h, b):
    # The gate/up tiles (both single-buffered forms) load two groups' scales
    # at once when both scale arrays are 4-byte aligned; 2-byte aligned
    # scales take 2-byte loads and give the same bits. At I <= 4096 the
    # aligned scales take the double-buffered tiles, which stage pairs only,
    # so there 2-byte aligned scales run the single-buffered tiles (another
    # order of the groups): both meet the oracle.
    from decode_kernel import _abi

    lib = _abi.load()
    (gp, gs, up, us, _, _), (ngp, ngs, nup, nus, _, _) = _weights(i, h, seed=i + b)
    x = _x(b, h, seed=b)
    stream = torch.cuda.current_stream().cuda_stream

    def shifted(t):
        buf = torch.empty(t.numel() + 1, dtype=torch.float16, device="cuda")
        buf[1:] = t.reshape(-1)
        assert buf[1:].data_ptr() % 4 == 2
        return buf

    def call(gsp, usp):
        hk = torch.empty(b, i, dtype=torch.float16, device="cuda")
        _abi.check(lib, lib.dk_gate_up_silu(gp.data_ptr(), gsp, up.data_ptr(), usp, x.data_ptr(),
                                            hk.data_ptr(), i, h, b, stream))
        return hk

    g2, u2 = shifted(gs), shifted(us)
    h_shifted = call(g2[1:].data_ptr(), u2[1:].data_ptr())
    h_aligned = call(gs.data_ptr(), us.data_ptr())
    if i > 4096:
        assert torch.equal(h_shifted, h_aligned)
    else:
        # Half an fp16 ulp of |h| + 1e-3 per output (|h| reaches ~32 here,
        # where one ulp is 0.03, above _check_tight's absolute gate).
        h_ref = oracle.gate_up_silu_f64(x.cpu().numpy(), ngp, ngs, nup, nus)
        for got, label in ((h_aligned, "aligned"), (h_shifted, "shifted")):
            err = np.abs(got.float().cpu().numpy().astype(np.float64) - h_ref)
            assert (err <= 0.5 * oracle.fp16_ulp(h_ref) + 1e-3).all(), f"h {i}x{h} B={b} {label}"
