// Fused gate/up projection of a Llama-style MLP decode step (SwiGLU):
//
//   h[b, i] = fp16( silu(g) * u ),  g = sum_k Wg[i, k] x[b, k],
//                                   u = sum_k Wu[i, k] x[b, k],
//   silu(v) = v / (1 + exp(-v)),
//
// with Wg and Wu in the W4A16 format of the GEMV (int4, group 128, fp16
// scales), g and u accumulated in fp32 exactly as the v5 GEMV accumulates a
// row, and the SiLU and product evaluated in fp32 before the one rounding to
// fp16. The down projection that follows is the v5 GEMV with h as its
// activations.
//
// No counterpart in the reference, which times one GEMV at a time: this is
// the step either side of its gemv() (python/decode_kernel/__init__.py:32-83)
// in a decoder's MLP. Fusing gate and up into one kernel shares each
// activation load and its fp16 pairing between the two matrices, and the
// SiLU*mul epilogue costs no extra launch or round trip of g and u.
//
// Mapping: the v5 streaming kernel with 2R rows per wave, rows 0..R-1 of the
// stage taken from Wg and rows R..2R-1 from Wu at the same row indices.
#pragma once

#include "dk_kernels.hpp"

namespace dk {

constexpr int kStampGateUp = 20;

__device__ __forceinline__ float silu_f32(float v) { return v / (1.0f + expf(-v)); }

template <int R, int U, int NB>
__global__ __launch_bounds__(kStreamWaves * 64) void gate_up_silu(const uint4* __restrict__ gate,
                                                    const uint16_t* __restrict__ gate_scales,
                                                    const uint4* __restrict__ up,
                                                    const uint16_t* __restrict__ up_scales,
                                                    const uint4* __restrict__ x4, int I, int H,
                                                    int B, uint16_t* __restrict__ h) {
  // h is the last argument: with 15 argument dwords not all fit the preload
  // registers, and h is only needed after the sums.
  write_stamp(kStampGateUp);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // The grid size follows from I (it is the launch's), so no hidden argument
  // is read before the first load.
  const int wg = xcd_contiguous_block(blockIdx.x, (I + kStreamWaves * R - 1) / (kStreamWaves * R));
  const int row0 = (wg * kStreamWaves + wave) * R;
  if (row0 >= I) return;  // wave-uniform; no barriers in this kernel
  const int b0 = blockIdx.y * NB;
  const int nck = H >> 5;
  const int G = H >> 7;
  const int rows = min(R, I - row0);
  const auto rwg = buffer_rsrc(gate + (size_t)row0 * nck, (uint32_t)(rows * (H / 2)));
  const auto rsg = buffer_rsrc(gate_scales + (size_t)row0 * G, (uint32_t)(rows * G * 2));
  const auto rwu = buffer_rsrc(up + (size_t)row0 * nck, (uint32_t)(rows * (H / 2)));
  const auto rsu = buffer_rsrc(up_scales + (size_t)row0 * G, (uint32_t)(rows * G * 2));
  const auto rx = buffer_rsrc(x4, (uint32_t)((size_t)B * H * 2));

  float acc[NB][2 * R];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int r = 0; r < 2 * R; ++r) acc[b][r] = 0.f;

  constexpr int kStep = U * kWave;
  V5Stage<2 * R, U, NB> st;
  for (int c0 = 0; c0 < nck; c0 += kStep) {
    v5_load<2 * R, U, NB, R>(st, rwg, rsg, rx, c0, nck, G, H, b0, B, lane, rwu, rsu);
    v5_compute(st, acc);
  }

#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float g = wave_sum(acc[b][r]);
      const float u = wave_sum(acc[b][R + r]);
      if (lane == 63 && row0 + r < I && b0 + b < B)
        h[(size_t)(b0 + b) * I + row0 + r] = f2h(silu_f32(g) * u);
    }
}

}  // namespace dk
