// STREAM-style HBM probes for MI355X: the read-only roof that is the
// denominator of the GEMV metric, plus copy and write for context, and an
// empty kernel for the per-launch floor.
// Reference: csrc/gemv_w4a16.cu:421-425 (copy), 493-551 (read, write),
// 593-626 (host wrappers).
//
// The read probe sums its buffer (DPP wave reduction) and writes one fp32
// partial per workgroup, so the loads cannot be eliminated.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "dk_device.hpp"
#include "dk_host.hpp"
#include "decode_kernel/dk_gemv.h"

namespace dk {

constexpr int kStreamThreads = 256;

// One 16-byte load per lane per grid-stride step. On MI355X this sustains a
// higher read rate (6.7+ TB/s over 1 GiB) than keeping 2-8 loads per lane in
// flight, which measured 5-20% slower.
__global__ __launch_bounds__(kStreamThreads) void stream_read_kernel(const float4* __restrict__ src,
                                                                     float* __restrict__ partials,
                                                                     size_t n) {
  __shared__ float wsum[kStreamThreads / 64];
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  float a = 0.f;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float4 v = src[i];
    a += (v.x + v.y) + (v.z + v.w);
  }
  a = wave_sum(a);
  const int lane = threadIdx.x & 63;
  if (lane == 63) wsum[threadIdx.x >> 6] = a;
  __syncthreads();
  if (threadIdx.x == 0) {
    float s = 0.f;
    for (int w = 0; w < kStreamThreads / 64; ++w) s += wsum[w];
    partials[blockIdx.x] = s;
  }
}

__global__ __launch_bounds__(kStreamThreads) void stream_write_kernel(float4* __restrict__ dst,
                                                                      size_t n) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  const float4 one = make_float4(1.f, 1.f, 1.f, 1.f);
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = one;
}

__global__ __launch_bounds__(kStreamThreads) void stream_copy_kernel(const float4* __restrict__ src,
                                                                     float4* __restrict__ dst,
                                                                     size_t n) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

__global__ void empty_kernel() {}

}  // namespace dk

extern "C" {

int dk_stream_recommended_blocks(void) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return -dk::hip_error(e, "hipGetDevice");
  int cus = 0;
  e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return -dk::hip_error(e, "hipDeviceGetAttribute");
  return std::max(1024, std::min(cus * 32, 8192));
}

int dk_stream_read(const void* src, float* partials, size_t bytes, int blocks, hipStream_t stream) {
  if (!src || !partials) return dk::set_error(DK_ERR_INVALID_ARGUMENT, "src and partials must not be NULL");
  if (bytes % 16 != 0) return dk::set_error(DK_ERR_INVALID_ARGUMENT, "buffer size must be a multiple of 16");
  if (reinterpret_cast<uintptr_t>(src) % 16 != 0)
    return dk::set_error(DK_ERR_INVALID_ARGUMENT, "src must be 16-byte aligned");
  if (blocks < 1) {
    blocks = dk_stream_recommended_blocks();
    if (blocks < 0) return -blocks;
  }
  hipLaunchKernelGGL(dk::stream_read_kernel, dim3(blocks), dim3(dk::kStreamThreads), 0, stream,
                     static_cast<const float4*>(src), partials, bytes / 16);
  return dk::check_launch("stream_read launch");
}

int dk_stream_write(void* dst, size_t bytes, int blocks, hipStream_t stream) {
  if (!dst) return dk::set_error(DK_ERR_INVALID_ARGUMENT, "dst must not be NULL");
  if (bytes % 16 != 0) return dk::set_error(DK_ERR_INVALID_ARGUMENT, "buffer size must be a multiple of 16");
  if (reinterpret_cast<uintptr_t>(dst) % 16 != 0)
    return dk::set_error(DK_ERR_INVALID_ARGUMENT, "dst must be 16-byte aligned");
  if (blocks < 1) {
    blocks = dk_stream_recommended_blocks();
    if (blocks < 0) return -blocks;
  }
  hipLaunchKernelGGL(dk::stream_write_kernel, dim3(blocks), dim3(dk::kStreamThreads), 0, stream,
                     static_cast<float4*>(dst), bytes / 16);
  return dk::check_launch("stream_write launch");
}

int dk_d2d_copy(const void* src, void* dst, size_t bytes, hipStream_t stream) {
  if (!src || !dst) return dk::set_error(DK_ERR_INVALID_ARGUMENT, "src and dst must not be NULL");
  if (bytes % 16 != 0) return dk::set_error(DK_ERR_INVALID_ARGUMENT, "copy size must be a multiple of 16");
  if (reinterpret_cast<uintptr_t>(src) % 16 != 0 || reinterpret_cast<uintptr_t>(dst) % 16 != 0)
    return dk::set_error(DK_ERR_INVALID_ARGUMENT, "src and dst must be 16-byte aligned");
  if (bytes == 0) return DK_OK;
  int blocks = dk_stream_recommended_blocks();
  if (blocks < 0) return -blocks;
  const size_t n = bytes / 16;
  const size_t need = (n + dk::kStreamThreads - 1) / dk::kStreamThreads;
  blocks = (int)std::min<size_t>((size_t)blocks, std::max<size_t>(need, 1));
  hipLaunchKernelGGL(dk::stream_copy_kernel, dim3(blocks), dim3(dk::kStreamThreads), 0, stream,
                     static_cast<const float4*>(src), static_cast<float4*>(dst), n);
  return dk::check_launch("d2d_copy launch");
}

int dk_empty_kernel(hipStream_t stream) {
  hipLaunchKernelGGL(dk::empty_kernel, dim3(1), dim3(64), 0, stream);
  return dk::check_launch("empty kernel launch");
}

}  // extern "C"
