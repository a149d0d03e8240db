// Symmetric group-128 int4 quantize-and-pack on the GPU, bit-exact with the
// reference quantizer (python/decode_kernel/quantize.py:26-51) on fp32 input.
//
// One thread per packed word (8 consecutive weights, two 16-byte loads). The
// 16 words of a 128-weight group are 16 consecutive lanes, which on gfx950 is
// one DPP row, so the group's amax is a 4-step DPP max inside the row. Then,
// per weight, exactly the reference's fp32 arithmetic: scale = amax / 7
// (correctly rounded division), clamped below at fp32(1e-8);
// q = clamp(rint_half_even(w / scale), -7, 7); nibble n of the word is
// q & 0xF at bit 4n; the scale is stored rounded to fp16 (round to nearest
// even). Reads 4 B and writes 0.5 B (+2 B per 128) per weight: HBM-bound.
#include <hip/hip_runtime.h>

#include "dk_device.hpp"
#include "dk_host.hpp"
#include "decode_kernel/dk_gemv.h"

namespace dk {

__device__ __forceinline__ float group_max16(float v) {
  v = fmaxf(v, dpp<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp<0x141>(v));  // row_half_mirror
  v = fmaxf(v, dpp<0x140>(v));  // row_mirror: all 16 lanes of the row
  return v;
}

__device__ __forceinline__ uint32_t nibble(float w, float scale, int n) {
  float q = rintf(w / scale);
  q = fminf(fmaxf(q, -7.0f), 7.0f);
  return ((uint32_t)(int)q & 0xFu) << (4 * n);
}

__global__ __launch_bounds__(256) void quantize_pack_kernel(const float4* __restrict__ w,
                                                            uint32_t* __restrict__ packed,
                                                            uint16_t* __restrict__ scales,
                                                            long long words) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const bool ok = i < words;
  const float4 a = ok ? w[2 * i] : make_float4(0.f, 0.f, 0.f, 0.f);
  const float4 b = ok ? w[2 * i + 1] : make_float4(0.f, 0.f, 0.f, 0.f);
  float m = fmaxf(fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))),
                  fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w))));
  // Groups are 16-word aligned and `words` is a multiple of 16, so a DPP row
  // is either one whole valid group or entirely past the end.
  m = group_max16(m);
  const float scale = fmaxf(m / 7.0f, 1e-8f);
  const uint32_t word = nibble(a.x, scale, 0) | nibble(a.y, scale, 1) | nibble(a.z, scale, 2) |
                        nibble(a.w, scale, 3) | nibble(b.x, scale, 4) | nibble(b.y, scale, 5) |
                        nibble(b.z, scale, 6) | nibble(b.w, scale, 7);
  if (!ok) return;
  packed[i] = word;
  if ((i & 15) == 0) scales[i >> 4] = f2h(scale);
}

// Reference word (nibble n at bits 4n) <-> paired word (even nibbles in the
// low half, odd nibbles in the high half, in order): a fixed permutation of
// the eight two's-complement nibbles.
__device__ __forceinline__ uint32_t to_paired(uint32_t w) {
  uint32_t p = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    p |= ((w >> (8 * j)) & 0xFu) << (4 * j);
    p |= ((w >> (8 * j + 4)) & 0xFu) << (16 + 4 * j);
  }
  return p;
}

__device__ __forceinline__ uint32_t from_paired(uint32_t p) {
  uint32_t w = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    w |= ((p >> (4 * j)) & 0xFu) << (8 * j);
    w |= ((p >> (16 + 4 * j)) & 0xFu) << (8 * j + 4);
  }
  return w;
}

template <bool kToPaired>
__global__ __launch_bounds__(256) void repack_kernel(const uint4* __restrict__ src,
                                                     uint4* __restrict__ dst, long long n4) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n4) return;
  uint4 v = src[i];
  if (kToPaired) {
    v = make_uint4(to_paired(v.x), to_paired(v.y), to_paired(v.z), to_paired(v.w));
  } else {
    v = make_uint4(from_paired(v.x), from_paired(v.y), from_paired(v.z), from_paired(v.w));
  }
  dst[i] = v;
}

}  // namespace dk

namespace {

template <bool kToPaired>
int repack(const uint32_t* src, uint32_t* dst, int M, int K, hipStream_t stream) {
  if (M < 0 || K < 0) return dk::set_error(DK_ERR_INVALID_ARGUMENT, "M and K must be >= 0");
  if (M == 0 || K == 0) return DK_OK;
  if (K % DK_GROUP_SIZE != 0)
    return dk::set_error(DK_ERR_INVALID_ARGUMENT, "K=%d is not divisible by group_size=128", K);
  if (!src || !dst) return dk::set_error(DK_ERR_INVALID_ARGUMENT, "src and dst must not be NULL");
  if (reinterpret_cast<uintptr_t>(src) % 16 != 0 || reinterpret_cast<uintptr_t>(dst) % 16 != 0)
    return dk::set_error(DK_ERR_INVALID_ARGUMENT, "src and dst must be 16-byte aligned");
  // K % 128 == 0, so every row is a whole number of 16-byte chunks.
  const long long n4 = (long long)M * (K / 32);
  const long long blocks = (n4 + 255) / 256;
  if (blocks > 0x7fffffffLL) return dk::set_error(DK_ERR_UNSUPPORTED, "M*K too large");
  hipLaunchKernelGGL(dk::repack_kernel<kToPaired>, dim3((unsigned)blocks), dim3(256), 0, stream,
                     reinterpret_cast<const uint4*>(src), reinterpret_cast<uint4*>(dst), n4);
  return dk::check_launch("repack launch");
}

}  // namespace

extern "C" int dk_repack_paired(const uint32_t* packed, uint32_t* paired, int M, int K,
                                hipStream_t stream) {
  return repack<true>(packed, paired, M, K, stream);
}

extern "C" int dk_unpack_paired(const uint32_t* paired, uint32_t* packed, int M, int K,
                                hipStream_t stream) {
  return repack<false>(paired, packed, M, K, stream);
}

extern "C" int dk_quantize_pack_f32(const float* w, int M, int K, uint32_t* packed,
                                    uint16_t* scales, hipStream_t stream) {
  if (M < 0 || K < 0) return dk::set_error(DK_ERR_INVALID_ARGUMENT, "M and K must be >= 0");
  if (M == 0 || K == 0) return DK_OK;
  if (K % DK_GROUP_SIZE != 0)
    return dk::set_error(DK_ERR_INVALID_ARGUMENT, "K=%d is not divisible by group_size=128", K);
  if (!w || !packed || !scales)
    return dk::set_error(DK_ERR_INVALID_ARGUMENT, "w, packed and scales must not be NULL");
  if (reinterpret_cast<uintptr_t>(w) % 16 != 0 || reinterpret_cast<uintptr_t>(packed) % 4 != 0 ||
      reinterpret_cast<uintptr_t>(scales) % 2 != 0)
    return dk::set_error(DK_ERR_INVALID_ARGUMENT,
                         "w must be 16-byte, packed 4-byte and scales 2-byte aligned");
  const long long words = (long long)M * (K / 8);
  const long long blocks = (words + 255) / 256;
  if (blocks > 0x7fffffffLL) return dk::set_error(DK_ERR_UNSUPPORTED, "M*K too large");
  hipLaunchKernelGGL(dk::quantize_pack_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                     reinterpret_cast<const float4*>(w), packed, scales, words);
  return dk::check_launch("quantize_pack launch");
}
