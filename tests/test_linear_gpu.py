"""GPU parity of the op API's second entry point and of the reference's C++
workspace contract.

* `w4a16_linear` (python/decode_kernel/__init__.py:62-83 of the reference):
  its default routing (the reuse path whenever more than one batch row is
  given, split_k 4 only for v4) checked by dispatch stamp and bit-equality
  with the explicit `gemv` call it stands for, and its output against the
  float64 oracle within half an fp16 ulp + 1e-3, at c0, c2 and c3 (B = 4, 16),
  with 1-D and 2-D activations.
* dk_w4a16_gemv_ref_workspace, the entry the reference-signature C++ wrapper
  (include/decode_kernel/gemv_w4a16.hpp) calls: v4 accumulates into a
  caller-zeroed fp32 [B, M] buffer (include/decode_kernel/gemv_w4a16.h:33 of
  the reference) and never writes past it; the buffer holds the fp32 sums
  afterwards; every other variant ignores it. A C++ program built against
  the header runs the same call on device buffers with a guard region (both
overloads run the same v4 kernel, so the same bits).
* The bench-only library's product-maths kernels compute the product's
  result (the ablation tool also checks this before timing), and its
  shader-clock probe reads a plausible SCLK.
"""

from __future__ import annotations

import ctypes
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import oracle

pytestmark = pytest.mark.gpu

REPO = Path(__file__).resolve().parents[1]


def _upload(m, k, b, seed):
    w, x = oracle.make_case(m, k, b, seed=seed)
    packed, scales = oracle.quantize_and_pack(w)
    return (packed, scales, x, torch.from_numpy(packed).cuda(), torch.from_numpy(scales).cuda(),
            torch.from_numpy(x).cuda())


def _tight(y: torch.Tensor, y_ref: np.ndarray, label: str):
    yk = y.float().cpu().numpy().astype(np.float64).reshape(y_ref.shape)
    err = np.abs(yk - y_ref)
    assert err.max() < 1e-2, f"{label}: max abs err {err.max():.3e}"
    bound = 0.5 * oracle.fp16_ulp(y_ref) + 1e-3
    assert (err <= bound).all(), f"{label}: {int((err > bound).sum())} outputs beyond half-ulp+1e-3"


@pytest.mark.parametrize("m,k,b", [(4096, 4096, 1), (4096, 11008, 1), (4096, 4096, 4),
                                   (4096, 4096, 16), (1000, 1024, 3)])
def test_w4a16_linear_routing_and_parity(m, k, b):
    from decode_kernel import _cuda, gemv, w4a16_linear

    packed, scales, x, pd, sd, xd = _upload(m, k, b, seed=500 + m + k + b)
    y_ref = oracle.linear_f64(x, packed, scales)
    print(f"[w4a16_linear] M={m} K={k} B={b}", flush=True)

    y = w4a16_linear(xd, pd, sd)
    stamp = _cuda.last_kernel_stamp()
    assert stamp == (5 if b == 1 else 15), stamp  # reuse whenever B > 1
    _tight(y, y_ref, f"w4a16_linear M={m} K={k} B={b}")
    y_explicit = gemv(pd, sd, xd, version=5, split_k=1, reuse_weights=b > 1)
    assert torch.equal(y, y_explicit)

    # version=4: split_k defaults to 4 (the result is bit-equal to the explicit
    # split_k=4 call: the split reduction is deterministic).
    y4 = w4a16_linear(xd, pd, sd, version=4)
    assert _cuda.last_kernel_stamp() == (4 if b == 1 else 15)
    _tight(y4, y_ref, f"w4a16_linear v4 M={m} K={k} B={b}")
    if b == 1:
        assert torch.equal(y4, gemv(pd, sd, xd, version=4, split_k=4))
    # Explicit arguments override the defaults.
    y4s = w4a16_linear(xd, pd, sd, version=4, split_k=2, reuse_weights=False)
    assert _cuda.last_kernel_stamp() == 4
    _tight(y4s, y_ref, f"w4a16_linear v4 sk2 M={m} K={k} B={b}")
    assert torch.equal(y4s, gemv(pd, sd, xd, version=4, split_k=2))
    y2 = w4a16_linear(xd, pd, sd, version=2, reuse_weights=False)
    assert _cuda.last_kernel_stamp() == 2
    _tight(y2, y_ref, f"w4a16_linear v2 M={m} K={k} B={b}")


def test_w4a16_linear_one_dimensional_x():
    from decode_kernel import _cuda, w4a16_linear

    packed, scales, x, pd, sd, xd = _upload(4096, 4096, 1, seed=42)
    y_ref = oracle.linear_f64(x, packed, scales)
    y = w4a16_linear(xd[0], pd, sd)  # [K] -> [1, M], streaming path (one row)
    assert y.shape == (1, 4096)
    assert _cuda.last_kernel_stamp() == 5
    _tight(y, y_ref, "w4a16_linear 1-D x")


def _ref_ws_call(lib, cfg, pd, sd, xd, m, k, b, ws):
    from decode_kernel import _abi

    y = torch.empty(b, m, dtype=torch.float16, device="cuda")
    rc = lib.dk_w4a16_gemv_ref_workspace(pd.data_ptr(), sd.data_ptr(), xd.data_ptr(), y.data_ptr(),
                                         m, k, b, ctypes.byref(cfg),
                                         ws.data_ptr() if ws is not None else None,
                                         torch.cuda.current_stream().cuda_stream)
    _abi.check(lib, rc)
    torch.cuda.synchronize()
    return y


@pytest.mark.parametrize("m,k,b,split", [(4096, 4096, 1, 4), (4096, 11008, 1, 4), (1000, 1024, 3, 4),
                                         (333, 640, 5, 32), (64, 128, 1, 1), (4096, 4096, 16, 8)])
def test_reference_workspace_v4(m, k, b, split):
    from decode_kernel import _abi

    lib = _abi.load()
    packed, scales, x, pd, sd, xd = _upload(m, k, b, seed=900 + m + b)
    y_ref = oracle.linear_f64(x, packed, scales)
    print(f"[ref workspace v4] M={m} K={k} B={b} split {split}", flush=True)
    cfg = _abi.default_config(lib, version=4, split_k=split)
    guard = 4096
    buf = torch.full((b * m + guard,), -7.25, dtype=torch.float32, device="cuda")
    buf[: b * m].zero_()
    for rep in range(2):  # the caller zeroes it before each call, as in the reference
        buf[: b * m].zero_()
        y = _ref_ws_call(lib, cfg, pd, sd, xd, m, k, b, buf)
        _tight(y, y_ref, f"ref-workspace v4 M={m} K={k} B={b} rep {rep}")
        assert bool((buf[b * m:] == -7.25).all()), "v4 wrote past the [B, M] workspace"
        acc = buf[: b * m].view(b, m)
        assert torch.equal(acc.half(), y), "workspace does not hold the fp32 sums of y"
    assert _cuda_stamp() == 4


def _cuda_stamp():
    from decode_kernel import _cuda

    return _cuda.last_kernel_stamp()


def test_reference_workspace_other_variants_ignore_it():
    from decode_kernel import _abi, gemv

    lib = _abi.load()
    m, k, b = 1000, 1024, 3
    _, _, _, pd, sd, xd = _upload(m, k, b, seed=31)
    for kw in (dict(version=5), dict(version=2), dict(version=1, warps_per_row=2),
               dict(version=5, reuse_weights=1)):
        cfg = _abi.default_config(lib, **kw)
        buf = torch.full((b * m + 64,), 3.5, dtype=torch.float32, device="cuda")
        y = _ref_ws_call(lib, cfg, pd, sd, xd, m, k, b, buf)
        assert torch.equal(y, gemv(pd, sd, xd, **{kk: v for kk, v in kw.items()})), kw
        assert bool((buf == 3.5).all()), f"{kw}: workspace touched"
        y0 = _ref_ws_call(lib, cfg, pd, sd, xd, m, k, b, None)
        assert torch.equal(y, y0), kw


CPP_GPU_PROGRAM = r"""
#include "decode_kernel/gemv_w4a16.hpp"
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <vector>
// The reference's C++ call pattern for v4 (a caller-zeroed fp32 [B, M]
// workspace, include/decode_kernel/gemv_w4a16.h:33), on device buffers with
// a guard region after the workspace, against the sized single-launch form.
int main() {
  using namespace decode_kernel;
  const int M = 777, K = 2304, B = 3, guard = 2048;
  std::vector<uint32_t> hp((size_t)M * K / 8);
  std::vector<__half> hs((size_t)M * K / 128), hx((size_t)B * K);
  uint32_t st = 12345u;
  auto next = [&]() { st = st * 1664525u + 1013904223u; return st; };
  for (auto& w : hp) w = next();
  for (auto& s : hs) s = __float2half(0.001f + (next() % 1000) * 1e-6f);
  for (auto& v : hx) v = __float2half(((int)(next() % 2001) - 1000) * 1e-3f);
  uint32_t* p; __half *s, *x, *y1, *y2; float* ws; void* ws2;
  if (hipMalloc(&p, hp.size() * 4) || hipMalloc(&s, hs.size() * 2) || hipMalloc(&x, hx.size() * 2) ||
      hipMalloc(&y1, (size_t)B * M * 2) || hipMalloc(&y2, (size_t)B * M * 2) ||
      hipMalloc(&ws, ((size_t)B * M + guard) * 4))
    return 10;
  if (hipMemcpy(p, hp.data(), hp.size() * 4, hipMemcpyHostToDevice) ||
      hipMemcpy(s, hs.data(), hs.size() * 2, hipMemcpyHostToDevice) ||
      hipMemcpy(x, hx.data(), hx.size() * 2, hipMemcpyHostToDevice))
    return 16;
  std::vector<float> sentinel((size_t)B * M + guard, -7.25f);
  std::fill(sentinel.begin(), sentinel.begin() + (size_t)B * M, 0.0f);
  if (hipMemcpy(ws, sentinel.data(), sentinel.size() * 4, hipMemcpyHostToDevice)) return 17;
  GemvLaunchConfig v4;
  v4.version = KernelVersion::V4;
  w4a16_gemv(p, s, x, y1, M, K, B, v4, ws, nullptr);  // the reference's signature
  const size_t bytes = workspace_bytes(M, K, B, v4);  // 0: v4 needs none
  ws2 = nullptr;
  if (bytes && hipMalloc(&ws2, bytes)) return 11;
  w4a16_gemv(p, s, x, y2, M, K, B, v4, ws2, bytes, nullptr);  // sized overload
  if (hipDeviceSynchronize() != hipSuccess) return 12;
  std::vector<float> after(sentinel.size());
  std::vector<__half> r1((size_t)B * M), r2((size_t)B * M);
  if (hipMemcpy(after.data(), ws, after.size() * 4, hipMemcpyDeviceToHost) ||
      hipMemcpy(r1.data(), y1, r1.size() * 2, hipMemcpyDeviceToHost) ||
      hipMemcpy(r2.data(), y2, r2.size() * 2, hipMemcpyDeviceToHost))
    return 18;
  for (size_t i = (size_t)B * M; i < after.size(); ++i)
    if (after[i] != -7.25f) { std::printf("guard overwritten at %zu\n", i); return 13; }
  double worst = 0;
  for (size_t i = 0; i < r1.size(); ++i) {
    const float a = __half2float(r1[i]), b = __half2float(r2[i]);
    const double tol = 1e-3 + std::ldexp(std::fabs(b), -10);
    worst = std::fmax(worst, std::fabs(a - b) / tol);
    if (__half2float(__float2half(after[i])) != a) { std::printf("ws[%zu] != y\n", i); return 14; }
    if (a != b) { std::printf("paths differ at %zu\n", i); return 19; }
  }
  if (worst > 1.0) { std::printf("paths differ: %.3f of tolerance\n", worst); return 15; }
  std::printf("ok %.3f\n", worst);
  return 0;
}
"""


def test_cpp_reference_signature_v4_on_device(tmp_path):
    if shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists():
        pytest.skip("hipcc not available")
    from decode_kernel import _abi

    src = tmp_path / "t.cpp"
    src.write_text(CPP_GPU_PROGRAM)
    exe = tmp_path / "t"
    libdir = _abi.LIB_PATH.parent
    subprocess.run(["g++", "-std=c++17", "-O1", "-D__HIP_PLATFORM_AMD__", f"-I{REPO / 'include'}",
                    "-I/opt/rocm/include", str(src), f"-L{libdir}", "-ldk_hip",
                    f"-Wl,-rpath,{libdir}", "-L/opt/rocm/lib", "-lamdhip64", "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=90)
    print(out.stdout, out.stderr, flush=True)
    assert out.returncode == 0 and out.stdout.startswith("ok"), (out.returncode, out.stdout)


def test_bench_library_variants_compute_the_gemv():
    from decode_kernel import _abi, _cuda
    from dk_bench import benchlib

    lib = _abi.load()
    for m, k in ((4096, 4096), (1000, 1024), (4096, 11008)):
        _, _, _, pd, sd, xd = _upload(m, k, 1, seed=77 + m)
        y_prod = _cuda.w4a16_gemv(pd, sd, xd)
        y = torch.empty_like(y_prod)
        kern = benchlib.parse_kernel(_abi.describe(lib, m, k, 1)["kernel"])
        for math in (0, 1, 2):
            # The ablation maths run the product's loads (their outputs are
            # not the GEMV); the product math is bit-equal to the product.
            benchlib.run_kernel(kern, math, pd, sd, xd, y)
        benchlib.run_kernel(kern, 0, pd, sd, xd, y)
        torch.cuda.synchronize()
        assert torch.equal(y, y_prod), (m, k, kern)


def test_shader_clock_probe():
    """The clock probe's SCLK (s_memtime cycles over s_memrealtime ticks)
    lies within MI355X's clock range, for one wave and for the whole chip."""
    from dk_bench import benchlib

    for blocks in (1, 1024):
        mhz = benchlib.sclk_mhz(iters=20000, blocks=blocks)
        assert 500.0 < mhz < 3000.0, (blocks, mhz)
