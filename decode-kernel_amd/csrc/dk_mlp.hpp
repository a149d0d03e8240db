// Fused gate/up projection of a Llama-style MLP decode step (SwiGLU):
//
//   h[b, i] = fp16( silu(g) * u ),  g = sum_k Wg[i, k] x[b, k],
//                                   u = sum_k Wu[i, k] x[b, k],
//   silu(v) = v / (1 + exp(-v)),
//
// with Wg and Wu in the W4A16 format of the GEMV (int4, group 128, fp16
// scales), g and u accumulated in fp32 exactly as the v5 GEMV accumulates a
// row, and the SiLU and product evaluated in fp32 before the one rounding to
// fp16. The down projection that follows is the GEMV with h as its
// activations (the weight-reuse path for a batch).
//
// No counterpart in the reference, which times one GEMV at a time: this is
// the step either side of its gemv() (python/decode_kernel/__init__.py:32-83)
// in a decoder's MLP. Fusing gate and up into one kernel shares each
// activation load and its fp16 pairing between the two matrices, and the
// SiLU*mul epilogue costs no extra launch or round trip of g and u.
//
// Mapping: the v5 streaming kernel with 2R rows per wave, rows 0..R-1 of the
// stage taken from Wg and rows R..2R-1 from Wu at the same row indices, so
// each activation stage in LDS serves both matrices; from 3 batch rows (4
// at I <= 4096 with H > 4096, 9 at I <= 2048, 17 at I <= 1024) the MFMA
// tiles of the reuse path, one tile of Wg and one of Wu per wave.
#pragma once

#include "dk_kernels.hpp"

namespace dk {

__device__ __forceinline__ float silu_f32(float v) { return v / (1.0f + expf(-v)); }

// The stage loop of gemv_v5_lds with NB batch rows per stage (grid.y covers
// the batch).
template <int R, int U, int W, int NB, bool kPrefetch>
__global__ __launch_bounds__(W * kWave) void gate_up_silu_lds(
    const uint4* __restrict__ gate, const uint16_t* __restrict__ gate_scales,
    const uint4* __restrict__ up, const uint16_t* __restrict__ up_scales,
    const uint4* __restrict__ x4, int I, int H, int B, uint16_t* __restrict__ h) {
  __shared__ LdsActs<U, NB> xs;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wg = xcd_contiguous_block(blockIdx.x, (I + W * R - 1) / (W * R));
  const int row0 = (wg * W + wave) * R;
  const bool active = row0 < I;  // wave-uniform; inactive waves still meet every barrier
  const int nck = H >> 5;
  const int G = H >> 7;
  const int rows = active ? min(R, I - row0) : 0;
  const int rbase = active ? row0 : 0;
  const auto rwg = buffer_rsrc(gate + (size_t)rbase * nck, (uint32_t)(rows * (H / 2)));
  const auto rsg = buffer_rsrc(gate_scales + (size_t)rbase * G, (uint32_t)(rows * G * 2));
  const auto rwu = buffer_rsrc(up + (size_t)rbase * nck, (uint32_t)(rows * (H / 2)));
  const auto rsu = buffer_rsrc(up_scales + (size_t)rbase * G, (uint32_t)(rows * G * 2));
  const auto rx = buffer_rsrc(x4, (uint32_t)((size_t)B * H * 2));
  const int b0 = blockIdx.y * NB;

  float acc[NB][2 * R];
  lds_stream<2 * R, U, W, NB, kPrefetch, LayoutLogical, R>(xs, acc, rwg, rsg, rwu, rsu, rx, nck, nck,
                                                            G, H, b0, B, tid, lane);
  if (!active) return;  // after the last barrier
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

// Batches of several rows: the MFMA tile loop of the GEMV's reuse path with
// its two tiles the same 16 rows of Wg and of Wu, so one activation load
// serves both matrices and each decoded weight serves up to 16 batch rows.
// The epilogue adds each tile's wave partials in wave order and forms h from
// the two fp32 sums, as the streaming kernel above does.
template <int KS, int SG, bool kPairs>
__global__ __launch_bounds__(KS * 64) void gate_up_silu_tiles(
    const uint4* __restrict__ gate, const uint16_t* __restrict__ gate_scales,
    const uint4* __restrict__ up, const uint16_t* __restrict__ up_scales,
    const uint4* __restrict__ x4, int I, int H, int B, uint16_t* __restrict__ h) {
  __shared__ ReuseLds<KS, 2, SG> lds;
  const int G = H >> 7;
  const int nck = H >> 5;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row0 = blockIdx.x * 16;
  const int b = blockIdx.y * kReuseBatch + (lane & 15);  // this lane's batch column
  const int kq = lane >> 4;
  const int rows = min(16, I - row0);
  const __amdgpu_buffer_rsrc_t rw[2] = {
      buffer_rsrc(gate + (size_t)row0 * nck, (uint32_t)(rows * (H / 2))),
      buffer_rsrc(up + (size_t)row0 * nck, (uint32_t)(rows * (H / 2)))};
  const __amdgpu_buffer_rsrc_t rs[2] = {
      buffer_rsrc(gate_scales + (size_t)row0 * G, (uint32_t)(rows * G * 2)),
      buffer_rsrc(up_scales + (size_t)row0 * G, (uint32_t)(rows * G * 2))};
  const auto rx = buffer_rsrc(x4, (uint32_t)((size_t)B * H * 2));
  const int xbase = b < B ? b * H * 2 + kq * 64 : kOutOfRange;
  f4_t acc[2];
  reuse_tile_loop<KS, 2, SG, kPairs>(acc, lds.wst[wave], rw, rs, rx, xbase, G, G, nck, lane, wave,
                                      b < B);
  reuse_tile_publish(lds, acc, wave, lane);
  __syncthreads();
  if (wave == 0) {
    const f4_t g = reuse_tile_sum(lds, 0, lane);
    const f4_t u = reuse_tile_sum(lds, 1, lane);
    if (b < B) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int orow = row0 + 4 * kq + v;
        if (orow < I) h[(size_t)b * I + orow] = f2h(silu_f32(g[v]) * u[v]);
      }
    }
  }
}

// The same with both tiles' operands staged in LDS by the buffer-load-to-LDS
// path (the GEMV's gemv_reuse_lds): tile 0 is 16 rows of Wg, tile 1 the
// same rows of Wu, one staged block of x serving both.
template <int KS, bool kPairs>
__global__ __launch_bounds__(KS * 64) void gate_up_silu_tiles_lds(
    const uint4* __restrict__ gate, const uint16_t* __restrict__ gate_scales,
    const uint4* __restrict__ up, const uint16_t* __restrict__ up_scales,
    const uint4* __restrict__ x4, int I, int H, int B, uint16_t* __restrict__ h) {
  __shared__ ReuseDmaLds<KS, 2> lds;
  const int G = H >> 7;
  const int nck = H >> 5;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row0 = blockIdx.x * 16;
  const int bt0 = blockIdx.y * kReuseBatch;
  const int b = bt0 + (lane & 15);  // this lane's batch column
  const int kq = lane >> 4;
  const int rows = __builtin_amdgcn_readfirstlane(min(16, I - row0));
  const __amdgpu_buffer_rsrc_t rw[2] = {
      buffer_rsrc(gate + (size_t)row0 * nck, (uint32_t)(rows * (H / 2))),
      buffer_rsrc(up + (size_t)row0 * nck, (uint32_t)(rows * (H / 2)))};
  const __amdgpu_buffer_rsrc_t rs[2] = {
      buffer_rsrc(gate_scales + (size_t)row0 * G, (uint32_t)(rows * G * 2)),
      buffer_rsrc(up_scales + (size_t)row0 * G, (uint32_t)(rows * G * 2))};
  const auto rx = buffer_rsrc(x4, (uint32_t)((size_t)B * H * 2));
  f4_t acc[2];
  reuse_lds_loop<KS, 2, kPairs>(acc, lds.x[wave], lds.w[wave], rw, rs, rx, bt0, B, H, G, lane,
                                wave);
  reuse_lds_publish(lds, acc, wave, lane);
  __syncthreads();
  if (wave == 0) {
    const f4_t g = reuse_lds_sum(lds, 0, lane);
    const f4_t u = reuse_lds_sum(lds, 1, lane);
    if (b < B) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int orow = row0 + 4 * kq + v;
        if (orow < I) h[(size_t)b * I + orow] = f2h(silu_f32(g[v]) * u[v]);
      }
    }
  }
}

// The same double buffered (the GEMV's gemv_reuse_pf): tiles 0 and 1 are
// 16 rows of Wg and Wu, each block's loads issued a block ahead, kXL x
// loads per block (batch tiles of up to 2 kXL rows: B <= 2 kXL or
// kXL = 8). Needs an even number of groups per row and 4-byte aligned
// scales.
template <int KS, int kXL = 8>
__global__ __launch_bounds__(KS * 64) void gate_up_silu_tiles_pf(
    const uint4* __restrict__ gate, const uint16_t* __restrict__ gate_scales,
    const uint4* __restrict__ up, const uint16_t* __restrict__ up_scales,
    const uint4* __restrict__ x4, int I, int H, int B, uint16_t* __restrict__ h) {
  __shared__ ReusePfLds<KS, 2, 2 * kXL> lds;
  const int G = H >> 7;
  const int nck = H >> 5;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row0 = blockIdx.x * 16;
  const int kq = lane >> 4;
  const int rows = __builtin_amdgcn_readfirstlane(min(16, I - row0));
  const __amdgpu_buffer_rsrc_t rw[2] = {
      buffer_rsrc(gate + (size_t)row0 * nck, (uint32_t)(rows * (H / 2))),
      buffer_rsrc(up + (size_t)row0 * nck, (uint32_t)(rows * (H / 2)))};
  const __amdgpu_buffer_rsrc_t rs[2] = {
      buffer_rsrc(gate_scales + (size_t)row0 * G, (uint32_t)(rows * G * 2)),
      buffer_rsrc(up_scales + (size_t)row0 * G, (uint32_t)(rows * G * 2))};
  const auto rx = buffer_rsrc(x4, (uint32_t)((size_t)B * H * 2));
  ReuseWindow win;
  win.bt0 = blockIdx.y * kReuseBatch;
  win.B = B;
  win.K = H;
  win.G = G;
  win.Gs = G;
  win.gbeg = 0;
  f4_t acc[2];
  reuse_pf_loop<KS, 2, kXL>(acc, lds, rw, rs, rx, win, lane, wave);
  reuse_pf_publish(lds, acc, wave, lane);
  __syncthreads();
  const int b = win.bt0 + (lane & 15);
  if (wave == 0) {
    const f4_t g = reuse_pf_sum(lds, 0, lane);
    const f4_t u = reuse_pf_sum(lds, 1, lane);
    if (b < B) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int orow = row0 + 4 * kq + v;
        if (orow < I) h[(size_t)b * I + orow] = f2h(silu_f32(g[v]) * u[v]);
      }
    }
  }
}

}  // namespace dk
