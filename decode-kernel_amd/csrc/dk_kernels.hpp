// Every W4A16 GEMV kernel for gfx950, as templates and __global__ functions.
// Included by exactly one translation unit of the library (dk_gemv.hip) and
// by the measurement library.
//
// Layout in HBM (the reference format, no repacking):
//   packed uint32 [M, K/8]: row m is K/2 bytes; 16-byte chunk c of a row holds
//                           weights k = 32c .. 32c+31 (4 words, low nibble first)
//   scales fp16  [M, K/128]: chunk c of row m uses scales[m, c/4]
//   x      fp16  [B, K], y fp16 [B, M]
#pragma once

#include <hip/hip_runtime.h>

#include "dk_device.hpp"
#include "decode_kernel/dk_gemv.h"

namespace dk {

// ---------------------------------------------------------------------------
// Dispatch stamps (the reference's numbering, csrc/gemv_w4a16.cu:18-25,74-368)
// are recorded by the host when a launch succeeds (dk_last_kernel_stamp);
// no kernel writes one. A template's kStamp names the stamp its launches
// record. (A stamp store from one thread of one workgroup, as the reference
// writes it, measured 0.04-0.05 us per launch on MI355X: 1.3% at M = K = 4096.)
// ---------------------------------------------------------------------------

// ---------------------------------------------------------------------------
// v0: one thread per row, scalar decode (the uncoalesced baseline stage).
// Reference: csrc/gemv_w4a16.cu:70-94.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void gemv_v0(const uint32_t* __restrict__ packed,
                                               const uint16_t* __restrict__ scales,
                                               const uint16_t* __restrict__ x,
                                               uint16_t* __restrict__ y, int M, int K, int B) {
  const int row = blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= M) return;
  const int words = K >> 3;
  const int G = K >> 7;
  const uint32_t* rw = packed + (size_t)row * words;
  const uint16_t* rs = scales + (size_t)row * G;
  for (int b = 0; b < B; ++b) {
    const uint16_t* xb = x + (size_t)b * K;
    float acc = 0.f;
    for (int i = 0; i < words; ++i) {
      const uint32_t w = rw[i];
      const float s = h2f(rs[i >> 4]);
#pragma unroll
      for (int n = 0; n < 8; ++n) {
        const int q = (int)(w << (28 - 4 * n)) >> 28;
        acc += s * (float)q * h2f(xb[8 * i + n]);
      }
    }
    y[(size_t)b * M + row] = f2h(acc);
  }
}

// ---------------------------------------------------------------------------
// v1: one wave64 per row; lane l reads words l, l+64, ... (256 contiguous
// bytes per wave instruction); one 16-byte x load per word.
// Reference: csrc/gemv_w4a16.cu:99-128.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void gemv_v1(const uint32_t* __restrict__ packed,
                                               const uint16_t* __restrict__ scales,
                                               const uint4* __restrict__ x4,
                                               uint16_t* __restrict__ y, int M, int K, int B) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= M) return;
  const int words = K >> 3;
  const int G = K >> 7;
  const uint32_t* rw = packed + (size_t)row * words;
  const uint16_t* rs = scales + (size_t)row * G;
  for (int b = 0; b < B; ++b) {
    const uint4* xb = x4 + (size_t)b * words;
    float acc = 0.f;
    for (int i = lane; i < words; i += kWave) {
      h2_t xp[4];
      pair_x(xb[i], xp);
      acc += h2f(rs[i >> 4]) * dot_word(rw[i], xp, 0.f);
    }
    acc = wave_sum(acc);
    if (lane == 63) y[(size_t)b * M + row] = f2h(acc);
  }
}

// ---------------------------------------------------------------------------
// v1 with K split over `wpr` waves of one workgroup per row, LDS reduction in
// wave order. Stamp 10 + wpr. Reference: csrc/gemv_w4a16.cu:134-172.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(512) void gemv_v1_multiwave(const uint32_t* __restrict__ packed,
                                                         const uint16_t* __restrict__ scales,
                                                         const uint4* __restrict__ x4,
                                                         uint16_t* __restrict__ y, int M, int K,
                                                         int B) {
  const int wpr = blockDim.x >> 6;
  __shared__ float red[8];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row = blockIdx.x;  // grid is exactly M
  const int words = K >> 3;
  const int G = K >> 7;
  const uint32_t* rw = packed + (size_t)row * words;
  const uint16_t* rs = scales + (size_t)row * G;
  for (int b = 0; b < B; ++b) {
    const uint4* xb = x4 + (size_t)b * words;
    float acc = 0.f;
    for (int i = wave * kWave + lane; i < words; i += wpr * kWave) {
      h2_t xp[4];
      pair_x(xb[i], xp);
      acc += h2f(rs[i >> 4]) * dot_word(rw[i], xp, 0.f);
    }
    acc = wave_sum(acc);
    if (lane == 63) red[wave] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
      float t = 0.f;
      for (int w = 0; w < wpr; ++w) t += red[w];
      y[(size_t)b * M + row] = f2h(t);
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// v2 / v3: one wave64 per row with 16-byte loads (32 weights per lane per
// load, 1 KiB per wave instruction). v3 stages the row's group scales in LDS.
// Reference: csrc/gemv_w4a16.cu:183-257.
// ---------------------------------------------------------------------------
template <bool kScalesInLds>
__global__ __launch_bounds__(256) void gemv_v23(const uint4* __restrict__ packed,
                                                const uint16_t* __restrict__ scales,
                                                const uint4* __restrict__ x4,
                                                uint16_t* __restrict__ y, int M, int K, int B) {
  extern __shared__ uint16_t lds_scales[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row_raw = blockIdx.x * (blockDim.x >> 6) + wave;
  const int row = row_raw < M ? row_raw : M - 1;  // clamp: keep waves alive for the barrier
  const int nck = K >> 5;
  const int G = K >> 7;
  const uint4* rw = packed + (size_t)row * nck;
  const uint16_t* rs = scales + (size_t)row * G;
  const uint16_t* sc = rs;
  if (kScalesInLds) {
    uint16_t* mine = lds_scales + wave * G;
    for (int g = lane; g < G; g += kWave) mine[g] = rs[g];
    __syncthreads();
    sc = mine;
  }
  for (int b = 0; b < B; ++b) {
    const uint4* xb = x4 + (size_t)b * (K >> 3);
    float acc = 0.f;
    for (int c = lane; c < nck; c += kWave) {
      const uint4 w = rw[c];
      float part = 0.f;
      h2_t xp[4];
      pair_x(xb[4 * c + 0], xp);
      part = dot_word(w.x, xp, part);
      pair_x(xb[4 * c + 1], xp);
      part = dot_word(w.y, xp, part);
      pair_x(xb[4 * c + 2], xp);
      part = dot_word(w.z, xp, part);
      pair_x(xb[4 * c + 3], xp);
      part = dot_word(w.w, xp, part);
      acc += h2f(sc[c >> 2]) * part;
    }
    acc = wave_sum(acc);
    if (lane == 63 && row_raw < M) y[(size_t)b * M + row] = f2h(acc);
  }
}

// ---------------------------------------------------------------------------
// Raw buffer loads for the streaming kernels: SGPR resource descriptors
// scoped to a wave's rows, so a chunk past the row end or a row past M is an
// out-of-range offset that reads 0 (tails need no branches and the loads
// issue back to back).
// ---------------------------------------------------------------------------
constexpr int kOutOfRange = (int)0x80000000;  // beyond any descriptor's num_records
constexpr int kLoadNonTemporal = 2;            // buffer-load cache policy bit "nt"

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  // dword3 = 0x00020000: raw (stride 0) 32-bit buffer on gfx9-family parts.
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

template <int kAux>
__device__ __forceinline__ uint4 buffer_load16(__amdgpu_buffer_rsrc_t r, int offset) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, kAux);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// ---------------------------------------------------------------------------
// v5: the streaming kernel (stamp 5, or the layout's). Each wave owns R
// consecutive rows; lane l owns 16-byte chunks l, l+64, ... of each of them,
// U chunks per lane per stage. A stage's loads are the activations, then
// the scales, then the weights with the non-temporal hint (read-once data).
// The activations of a stage (NB batch rows x U * 4 KiB) are loaded once per
// workgroup of W waves, one to four 16-byte loads per lane, paired once for
// the layout, and read by every wave from LDS. Loading them per wave instead
// (an earlier form of this kernel) re-reads twice the weight bytes from L2
// at two rows per wave and pairs them in every wave; that cost 4-21% at the
// shapes measured for one batch row and more with a batch.
// Workgroup ids are renumbered so each XCD streams one contiguous block of
// rows (measured 2-5% faster). Reference: csrc/gemv_w4a16.cu:318-357.
// Two LDS buffers alternate by stage, so one barrier per stage suffices: a
// wave writes buffer b at stage s only after every wave has passed the
// barrier of stage s-1, which each wave reaches after its reads of buffer b
// (stage s-2). Waves past M still load activations and meet every barrier.
// kPrefetch: the next stage's loads are issued before this stage's math, in
// a second register set (the loop is unrolled by two so that no register
// copy waits on a load, and the loads are unconditional, reading zeros past
// the row end, so the wait counts stay exact). It pays when few waves share
// a SIMD; with many rows the extra registers cost more occupancy than the
// overlap gains.
// grid.y covers the batch in tiles of NB rows.
// ---------------------------------------------------------------------------
// kS > 1 (split-K, v4): the stage holds kS U chunks per lane of activations
// and the kS waves of a row take U of them each (wave slice sl: stage chunks
// 64 (sl U + u) + l), so a row's chunks are dealt to its waves stage by stage.
template <int R, int U, int W, int NB, int kS = 1>
struct LdsStage {
  static constexpr int kPiecesPerRow = kS * U * 4 * kWave;  // 16-byte pieces of one batch row
  static constexpr int kPieces = NB * kPiecesPerRow;
  static constexpr int kPer = (kPieces + W * kWave - 1) / (W * kWave);
  uint4 xv[kPer];
  uint4 w[U][R];
  uint32_t s[U][R];  // raw fp16 scale bits, converted where used
};

// One stage's activations in LDS: slot ((b * U + u) * 4 + j) * 64 + l holds
// the pairs of bytes [16j, 16j + 16) of chunk c0 + 64u + l of batch row
// b0 + b.
template <int U, int NB>
struct LdsActsT {
  static constexpr int kSlots = NB * U * 4 * kWave;
  using type = uint4[2][kSlots];
};
template <int U, int NB>
using LdsActs = typename LdsActsT<U, NB>::type;

// Rows r < kSplit come from (rw, rs), rows r >= kSplit from (rw2, rs2) as
// their row r - kSplit (the fused gate/up kernel streams two matrices
// against one activation stage; the GEMV has kSplit = R).
template <int R, int U, int W, int NB, int kSplit, int kS = 1>
__device__ __forceinline__ void lds_stage_load(LdsStage<R, U, W, NB, kS>& st,
                                               __amdgpu_buffer_rsrc_t rw, __amdgpu_buffer_rsrc_t rs,
                                               __amdgpu_buffer_rsrc_t rw2,
                                               __amdgpu_buffer_rsrc_t rs2, __amdgpu_buffer_rsrc_t rx,
                                               int c0, int nck, int wstride, int G, int K, int b0,
                                               int B, int tid, int lane, int sl = 0) {
  using S = LdsStage<R, U, W, NB, kS>;
  // Activations of chunks [c0, c0 + 64 kS U) of batch row b0 + b: piece p of
  // that row is bytes [16p, 16p + 16) of the range, so consecutive lanes
  // read consecutive 16 bytes.
#pragma unroll
  for (int i = 0; i < S::kPer; ++i) {
    const int piece = tid + i * W * kWave;
    const int b = piece / S::kPiecesPerRow;
    const int p = piece % S::kPiecesPerRow;
    const int c = c0 + (p >> 2);
    const bool ok = piece < S::kPieces && c < nck && b0 + b < B;
    st.xv[i] = buffer_load16<0>(rx, ok ? (b0 + b) * K * 2 + (c0 * 4 + p) * 16 : kOutOfRange);
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int c = c0 + (sl * U + u) * kWave + lane;
    const bool ok = c < nck;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int rr = r < kSplit ? r : r - kSplit;
      st.s[u][r] = __builtin_amdgcn_raw_buffer_load_b16(
          r < kSplit ? rs : rs2, ok ? (rr * G + (c >> 2)) * 2 : kOutOfRange, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int rr = r < kSplit ? r : r - kSplit;
      st.w[u][r] = buffer_load16<kLoadNonTemporal>(r < kSplit ? rw : rw2,
                                                   ok ? (rr * wstride + c) * 16 : kOutOfRange);
    }
  }
}

// Pairs this lane's activation pieces for the layout and stores them where
// the lane that owns the chunk reads them (slot layout above). Lanes past
// the stage's pieces (workgroups of more than 4U * NB waves) have none; the
// test is uniform per wave, so those waves skip the store.
template <int R, int U, int W, int NB, typename Layout, int kS = 1>
__device__ __forceinline__ void lds_stage_publish(const LdsStage<R, U, W, NB, kS>& st,
                                                  uint4 (&xs)[LdsActsT<kS * U, NB>::kSlots],
                                                  int tid) {
  using S = LdsStage<R, U, W, NB, kS>;
#pragma unroll
  for (int i = 0; i < S::kPer; ++i) {
    const int piece = tid + i * W * kWave;
    if (S::kPieces % (W * kWave) == 0 || piece < S::kPieces) {
      const int b = piece / S::kPiecesPerRow;
      const int cr = (piece % S::kPiecesPerRow) >> 2;  // chunk within the stage: 64 u + l
      h2_t p[4];
      Layout::pair(st.xv[i], p);
      xs[((b * kS * U + cr / kWave) * 4 + (piece & 3)) * kWave + cr % kWave] =
          make_uint4(__builtin_bit_cast(uint32_t, p[0]), __builtin_bit_cast(uint32_t, p[1]),
                     __builtin_bit_cast(uint32_t, p[2]), __builtin_bit_cast(uint32_t, p[3]));
    }
  }
}

template <int R, int U, int W, int NB, typename Layout, int kS = 1>
__device__ __forceinline__ void lds_stage_compute(const LdsStage<R, U, W, NB, kS>& st,
                                                  const uint4 (&xs)[LdsActsT<kS * U, NB>::kSlots],
                                                  float (&acc)[NB][R], int lane, int sl = 0) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    h2_t xp[NB][4][4];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint4 pv = xs[((b * kS * U + sl * U + u) * 4 + j) * kWave + lane];
        xp[b][j][0] = as_h2(pv.x);
        xp[b][j][1] = as_h2(pv.y);
        xp[b][j][2] = as_h2(pv.z);
        xp[b][j][3] = as_h2(pv.w);
      }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t words[4] = {st.w[u][r].x, st.w[u][r].y, st.w[u][r].z, st.w[u][r].w};
      float part[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) part[b] = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        h2_t q[4];
        Layout::unpack(words[j], q);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          part[b] = __builtin_amdgcn_fdot2(q[0], xp[b][j][0], part[b], false);
          part[b] = __builtin_amdgcn_fdot2(q[1], xp[b][j][1], part[b], false);
          part[b] = __builtin_amdgcn_fdot2(q[2], xp[b][j][2], part[b], false);
          part[b] = __builtin_amdgcn_fdot2(q[3], xp[b][j][3], part[b], false);
        }
      }
      const float sc = h2f((uint16_t)st.s[u][r]);
#pragma unroll
      for (int b = 0; b < NB; ++b) acc[b][r] = __builtin_fmaf(part[b], sc, acc[b][r]);
    }
  }
}

// Workgroup barrier for the stage loop. The scheduling barriers keep ALU
// work on either side of it: left alone, the scheduler hoists the weight
// decode (pure ALU on loaded registers) above s_barrier, which makes the
// wave wait for its weights before the barrier instead of after it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);
}

// The decode and products of one stage (the default math of the stage loop).
struct StageMath {
  template <int R, int U, int W, int NB, typename Layout, int kS>
  static __device__ __forceinline__ void compute(const LdsStage<R, U, W, NB, kS>& st,
                                                 const uint4 (&xs)[LdsActsT<kS * U, NB>::kSlots],
                                                 float (&acc)[NB][R], int lane, int sl) {
    lds_stage_compute<R, U, W, NB, Layout, kS>(st, xs, acc, lane, sl);
  }
};

// The stage loop shared by the GEMV, split-K and the fused gate/up kernel:
// acc[b][r] is row r's fp32 sum for batch row b0 + b over this lane's chunks
// of [0, nck) (a whole row, or one K slice of it), or with kS > 1 over the
// chunks of slice sl (the U of every kS U per lane that are this wave's).
// Weight row r starts wstride chunks after row r - 1 in its descriptor;
// scales G entries; batch rows of x K elements.
template <int R, int U, int W, int NB, bool kPrefetch, typename Layout, int kSplit,
          typename Math = StageMath, int kS = 1>
__device__ __forceinline__ void lds_stream(LdsActs<kS * U, NB>& xs, float (&acc)[NB][R],
                                           __amdgpu_buffer_rsrc_t rw, __amdgpu_buffer_rsrc_t rs,
                                           __amdgpu_buffer_rsrc_t rw2, __amdgpu_buffer_rsrc_t rs2,
                                           __amdgpu_buffer_rsrc_t rx, int nck, int wstride, int G,
                                           int K, int b0, int B, int tid, int lane, int sl = 0) {
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[b][r] = 0.f;
  constexpr int kStep = kS * U * kWave;
  if constexpr (kPrefetch) {
    // Two register sets, the loop unrolled by two so that no register copy
    // waits on a load; the prefetch loads are unconditional (zeros past the
    // row end) so the wait counts stay exact. The compiler sinks the first
    // half's prefetch below the exit test, so only every other stage is
    // prefetched before the math. Taking stages in pairs (every prefetch
    // ahead of the math) measured 2-4% slower at 3-7 stages per row and 2%
    // faster at 14 (M = 8192, K = 28672). Workgroups with more lanes than
    // activation pieces keep the publish test: giving the spare lanes
    // padding slots instead (so every lane loads and stores) cost 11-17%.
    LdsStage<R, U, W, NB, kS> sa, sb;
    lds_stage_load<R, U, W, NB, kSplit, kS>(sa, rw, rs, rw2, rs2, rx, 0, nck, wstride, G, K, b0,
                                            B, tid, lane, sl);
    for (int c0 = 0;;) {
      lds_stage_publish<R, U, W, NB, Layout, kS>(sa, xs[0], tid);
      __syncthreads();
      lds_stage_load<R, U, W, NB, kSplit, kS>(sb, rw, rs, rw2, rs2, rx, c0 + kStep, nck, wstride,
                                              G, K, b0, B, tid, lane, sl);
      __builtin_amdgcn_sched_barrier(0);
      Math::template compute<R, U, W, NB, Layout, kS>(sa, xs[0], acc, lane, sl);
      c0 += kStep;
      if (c0 >= nck) break;
      lds_stage_publish<R, U, W, NB, Layout, kS>(sb, xs[1], tid);
      __syncthreads();
      lds_stage_load<R, U, W, NB, kSplit, kS>(sa, rw, rs, rw2, rs2, rx, c0 + kStep, nck, wstride,
                                              G, K, b0, B, tid, lane, sl);
      __builtin_amdgcn_sched_barrier(0);
      Math::template compute<R, U, W, NB, Layout, kS>(sb, xs[1], acc, lane, sl);
      c0 += kStep;
      if (c0 >= nck) break;
    }
  } else {
    LdsStage<R, U, W, NB, kS> st;
    int buf = 0;
    for (int c0 = 0; c0 < nck; c0 += kStep, buf ^= 1) {
      lds_stage_load<R, U, W, NB, kSplit, kS>(st, rw, rs, rw2, rs2, rx, c0, nck, wstride, G, K,
                                              b0, B, tid, lane, sl);
      // Every load of the stage issues before the publish waits on the
      // activation pieces (left alone, the scheduler can put that wait
      // between the loads).
      __builtin_amdgcn_sched_barrier(0);
      lds_stage_publish<R, U, W, NB, Layout, kS>(st, xs[buf], tid);
      lds_barrier();
      Math::template compute<R, U, W, NB, Layout, kS>(st, xs[buf], acc, lane, sl);
    }
  }
}

template <int R, int U, int W, int NB, bool kPrefetch, typename Layout = LayoutLogical,
          int kStamp = Layout::kStamp, typename Math = StageMath>
__global__ __launch_bounds__(W * kWave) void gemv_v5_lds(const uint4* __restrict__ packed,
                                                         const uint16_t* __restrict__ scales,
                                                         const uint4* __restrict__ x4,
                                                         uint16_t* __restrict__ y, int M, int K,
                                                         int B) {
  __shared__ LdsActs<U, NB> xs;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wg = xcd_contiguous_block(blockIdx.x, (M + W * R - 1) / (W * R));
  const int row0 = (wg * W + wave) * R;
  const bool active = row0 < M;  // wave-uniform
  const int b0 = blockIdx.y * NB;
  const int nck = K >> 5;
  const int G = K >> 7;
  // An inactive wave gets empty weight and scale descriptors: all its
  // weight and scale loads read zero.
  const int rows = active ? min(R, M - row0) : 0;
  const int rbase = active ? row0 : 0;
  const auto rw = buffer_rsrc(packed + (size_t)rbase * nck, (uint32_t)(rows * (K / 2)));
  const auto rs = buffer_rsrc(scales + (size_t)rbase * G, (uint32_t)(rows * G * 2));
  const auto rx = buffer_rsrc(x4, (uint32_t)((size_t)B * K * 2));

  float acc[NB][R];
  lds_stream<R, U, W, NB, kPrefetch, Layout, R, Math>(xs, acc, rw, rs, rw, rs, rx, nck, nck, G, K,
                                                      b0, B, tid, lane);
  if (!active) return;  // after the last barrier
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float t = wave_sum(acc[b][r]);
      if (lane == 63 && row0 + r < M && b0 + b < B) y[(size_t)(b0 + b) * M + row0 + r] = f2h(t);
    }
}

// ---------------------------------------------------------------------------
// Completion tickets of a split-K reduction across workgroups (the reuse
// path's split-K tiles): 64 bits, (generation << 6) | arrivals. The first
// arrival of a call replaces whatever the ticket held, so a workspace needs
// no clearing; the last resets it to (generation, 0), so graph replays of
// one captured call (same generation) start clean. Generations are 58 bits
// and never repeat in a process, so only a ticket holding this call's exact
// generation before the call (2^-58 for arbitrary memory) would be
// miscounted.
// ---------------------------------------------------------------------------
// Takes the ticket of a split reduction for generation `gen` (low 6 bits
// zero); true for the last of `S` arrivals. One thread per workgroup, after
// a workgroup barrier that follows every wave's partial stores.
//
// Ordering. Every access here and to the partials is a relaxed atomic at
// agent scope, so the HIP memory model alone does not order the partial
// stores before the ticket. The order rests on how gfx950 executes them
// (checked in this library's assembly):
//  1. each partial is stored by `global_store_dword ... sc1` (agent scope:
//     written through the issuing XCD's L2), and every wave executes
//     `s_waitcnt vmcnt(0)` (reuse_split_finish) before the workgroup's
//     `s_barrier`, so the stores are acknowledged before the ticket is taken;
//  2. the ticket is a `global_atomic_cmpswap_x2` at agent scope, performed at
//     the device-coherent level, which serializes the S arrivals;
//  3. the last arrival's partial loads are `global_load_dword ... sc1` (agent
//     scope: they miss the XCD's L2 and read the coherent copy), issued only
//     after the compare-and-swap has returned and a barrier has passed.
// The formal alternative, an acquire-release compare-and-swap, makes the
// compiler write back the XCD's L2 before it and invalidate the L2 after it
// in every workgroup; measured on MI355X it cost 10-46% at the split shapes
// (M = 1024, K = 28672, B = 16: 21.7 against 14.8 us) with identical bits,
// so the relaxed form stays.
__device__ __forceinline__ bool take_ticket(unsigned long long* ticket, unsigned long long gen, int S) {
  unsigned long long t = __hip_atomic_load(ticket, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  unsigned long long arrived;
  for (;;) {
    arrived = (t & ~63ull) == gen ? (t & 63ull) : 0ull;
    // On failure t holds the current value; the loop ends when this
    // workgroup's increment lands (at most S workgroups contend).
    if (__hip_atomic_compare_exchange_strong(ticket, &t, gen | (arrived + 1ull), __ATOMIC_RELAXED,
                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
      break;
  }
  return arrived == (unsigned long long)(S - 1);
}

__device__ __forceinline__ void release_ticket(unsigned long long* ticket, unsigned long long gen) {
  __hip_atomic_store(ticket, gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// v4, split-K (stamp 4): the streaming kernel with each row taken by kS
// waves of its workgroup. The workgroup's W waves are W / kS row waves of R
// rows times kS slices (wave w: slice w / (W / kS), rows of row wave
// w % (W / kS)); each stage holds kS U chunks per lane of activations, and
// the wave of slice sl takes U of them (stage chunks 64 (sl U + u) + l), so
// the kS waves of a row share its stages' loads and the stage loop,
// prefetch and single barrier per stage are the GEMV's. After the last stage
// each wave's row sums go to LDS and the slice-0 wave of each row adds the
// kS of them in slice order (deterministic; fixed for a launch shape) and
// writes y, and the fp32 sums to `acc` when one is given (the reference's
// workspace contract). One launch, no workspace: the slices meet inside one
// CU. kS = 1 is the GEMV. Its launches record stamp 4 for v4, 5 where the
// v5 dispatch takes this kernel (it is faster than gemv_v5_lds at some
// shapes).
// ---------------------------------------------------------------------------
template <int R, int U, int W, int kS, int NB, bool kPrefetch, typename Math = StageMath>
__global__ __launch_bounds__(W * kWave) void gemv_v4_split(const uint4* __restrict__ packed,
                                                           const uint16_t* __restrict__ scales,
                                                           const uint4* __restrict__ x4,
                                                           uint16_t* __restrict__ y,
                                                           float* __restrict__ acc_out, int M,
                                                           int K, int B) {
  static_assert(W % kS == 0, "a workgroup holds whole rows");
  constexpr int kRowWaves = W / kS;
  constexpr int kRows = kRowWaves * R;  // rows per workgroup
  __shared__ LdsActs<kS * U, NB> xs;
  __shared__ float red[kS > 1 ? kS * NB * kRows : 1];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int sl = wave / kRowWaves;
  const int rwave = wave % kRowWaves;
  const int wg = xcd_contiguous_block(blockIdx.x, (M + kRows - 1) / kRows);
  const int row0 = wg * kRows + rwave * R;
  const bool active = row0 < M;  // wave-uniform
  const int b0 = blockIdx.y * NB;
  const int nck = K >> 5;
  const int G = K >> 7;
  const int rows = active ? min(R, M - row0) : 0;
  const int rbase = active ? row0 : 0;
  const auto rw = buffer_rsrc(packed + (size_t)rbase * nck, (uint32_t)(rows * (K / 2)));
  const auto rs = buffer_rsrc(scales + (size_t)rbase * G, (uint32_t)(rows * G * 2));
  const auto rx = buffer_rsrc(x4, (uint32_t)((size_t)B * K * 2));

  float acc[NB][R];
  lds_stream<R, U, W, NB, kPrefetch, LayoutLogical, R, Math, kS>(
      xs, acc, rw, rs, rw, rs, rx, nck, nck, G, K, b0, B, tid, lane, sl);
  if constexpr (kS == 1) {
    if (!active) return;  // after the last barrier
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float t = wave_sum(acc[b][r]);
        if (lane == 63 && row0 + r < M && b0 + b < B) {
          const size_t o = (size_t)(b0 + b) * M + row0 + r;
          y[o] = f2h(t);
          if (acc_out) acc_out[o] = t;
        }
      }
  } else {
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float t = wave_sum(acc[b][r]);
        if (lane == 63) red[(sl * NB + b) * kRows + rwave * R + r] = t;
      }
    __syncthreads();
    // Lane b R + r of the slice-0 wave adds row row0 + r's sums for batch
    // row b0 + b.
    if (sl == 0 && active && lane < NB * R) {
      const int b = lane / R;
      const int r = lane % R;
      if (row0 + r < M && b0 + b < B) {
        float sum = 0.f;
#pragma unroll
        for (int s2 = 0; s2 < kS; ++s2) sum += red[(s2 * NB + b) * kRows + rwave * R + r];
        const size_t o = (size_t)(b0 + b) * M + row0 + r;
        y[o] = f2h(sum);
        if (acc_out) acc_out[o] = sum;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Weight-reuse path (stamp 15): each decoded weight is used for up to 16
// batch rows at once by v_mfma_f32_16x16x32_f16, so latency is nearly flat
// in B instead of the reference's O(B) re-decode (csrc/gemv_w4a16.cu:364-413).
// A workgroup of KS waves owns RT 16-row tiles (one or two; with two, each
// activation load serves both); wave w takes the blocks of SG consecutive
// groups (two in every shape used) starting at groups SG w, SG (w + KS), ...
// The MFMA operands:
//   A (16x32, weights): lane l -> row l%16, 8 k-slots of lane group l/16
//   B (32x16, x):       lane l -> batch l%16, same 8 k-slots
//   D (16x16):          lane l -> rows 4(l/16)+v, batch l%16
// Lane l's A operand for group g is row l%16, bytes [64g + 16(l/16), +16):
// four words = four MFMA k-steps that together cover exactly group g, so
// the fp32 tile result of a group is scaled once and accumulated. Loading
// those 16 bytes directly (one instruction reads 64 bytes from each of 16
// rows) is slow at long rows; instead each block's weights come in
// instructions of 64 / (4 SG) rows x 64 SG contiguous bytes (8 rows x 128
// bytes for two groups), go through a wave-private LDS buffer (one pad slot
// per row against bank conflicts) and are read back in the A layout.
// Measured against the direct loads on MI355X: 8-20% faster at M = 11008 or
// K = 28672 and 3-8% at M = K = 4096 for 5-16 batch rows. Each lane loads
// the scales of its four D rows directly (a block's two groups in one 4-byte
// load where the scales allow). Each wave stores its partials over its own
// staging buffer and the KS of them are added in wave order. Loads are raw
// buffer loads through wave-uniform descriptors; rows past M, groups past G
// and batch rows past B read zero through out-of-range offsets.
// For up to two batch rows (three below 2^27 weights unless rows of
// 4097-8191 weights and M >= 3072, four below M = 3072),
// and more at small M (up to 8 rows at M <= 2048, 16 at M <= 1024, 32 at
// M <= 512, any at M <= 128), the reuse path runs the streaming kernel above
// instead (each decoded weight still serves every batch row of its tile):
// 16 MFMA batch columns cost more activation traffic than they save at small
// batches, and M / 16 tiles leave most CUs idle at small M.
// ---------------------------------------------------------------------------
constexpr int kReuseBatch = 16;

// The wave's own LDS traffic is ordered by these fences (no workgroup barrier:
// every buffer is private to one wave).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The block loop of the tile kernels: KS waves per workgroup, RT 16-row
// tiles per wave sharing each activation load (tile t's weights and scales
// through descriptors rw[t], rs[t], rows 0..15 relative to them, starting at
// the first of the G groups covered; a row's scales are Gstride apart), SG
// consecutive groups per block. acc[t] is this lane's part of tile t's fp32
// 16x16 result over the wave's blocks. kPairs (two groups per block, an even
// number of groups per row, 4-byte aligned scales): one 4-byte load brings
// the scales of both groups of a block, which takes a lane's scale registers
// from 4 * RT * SG to 4 * RT.
template <int KS, int RT, int SG, bool kPairs = false>
__device__ __forceinline__ void reuse_tile_loop(f4_t (&acc)[RT], uint4* wbuf,
                                                const __amdgpu_buffer_rsrc_t (&rw)[RT],
                                                const __amdgpu_buffer_rsrc_t (&rs)[RT],
                                                __amdgpu_buffer_rsrc_t rx, int xbase, int G,
                                                int Gstride, int nck, int lane, int wave,
                                                bool batch_ok) {
  static_assert(SG == 2 || SG == 4, "a block is two or four groups");
  static_assert(!kPairs || SG == 2, "paired scales take blocks of two groups");
  constexpr int kSlots = SG * 4 + 1;    // 16-byte slots per staged row, one of them padding
  constexpr int kLanesPerRow = SG * 4;  // lanes loading one row's block
  constexpr int kRowsPerLoad = 64 / kLanesPerRow;
  constexpr int kLoads = 16 * RT / kRowsPerLoad;
  constexpr int kLoadsPerTile = 16 / kRowsPerLoad;
  const int r_lane = lane & 15;
  const int kq = lane >> 4;
  const int lrow = lane / kLanesPerRow;  // row within one staging load
  const int lcol = lane % kLanesPerRow;  // 16-byte slot within the row's block
#pragma unroll
  for (int t = 0; t < RT; ++t) acc[t] = f4_t{0.f, 0.f, 0.f, 0.f};
  for (int g0 = SG * wave; g0 < G; g0 += SG * KS) {
    // Weights of groups g0..g0+SG-1: load i reads rows kRowsPerLoad * i +
    // lrow of the workgroup's 16 RT rows (tile i / kLoadsPerTile), lane lcol
    // taking bytes [16 lcol, +16) of the row's block.
    const int run = g0 * 64 + lcol * 16;
    uint4 wl[kLoads];
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int r = (i % kLoadsPerTile) * kRowsPerLoad + lrow;
      wl[i] = buffer_load16<kLoadNonTemporal>(rw[i / kLoadsPerTile],
                                              run < G * 64 ? r * nck * 16 + run : kOutOfRange);
    }
    uint4 xv[SG][4];
    float sc[RT][kPairs ? 1 : SG][4];
    uint32_t sc2[RT][kPairs ? 4 : 1];
#pragma unroll
    for (int u = 0; u < SG; ++u) {
      const int g = g0 + u;
      const int xo = (batch_ok && g < G) ? xbase + g * 256 : kOutOfRange;
#pragma unroll
      for (int j = 0; j < 4; ++j) xv[u][j] = buffer_load16<0>(rx, xo + 16 * j);
    }
#pragma unroll
    for (int t = 0; t < RT; ++t) {
      if constexpr (kPairs) {
        // g0 is even and G is even, so g0 + 1 < G as well.
#pragma unroll
        for (int v = 0; v < 4; ++v)
          sc2[t][v] = __builtin_amdgcn_raw_buffer_load_b32(rs[t], ((4 * kq + v) * Gstride + g0) * 2, 0, 0);
      } else {
#pragma unroll
        for (int u = 0; u < SG; ++u) {
          const int g = g0 + u;
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int off = g < G ? ((4 * kq + v) * Gstride + g) * 2 : kOutOfRange;
            sc[t][u][v] = h2f(__builtin_amdgcn_raw_buffer_load_b16(rs[t], off, 0, 0));
          }
        }
      }
    }
    // Every load of the block issues before the first wait.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < kLoads; ++i) wbuf[(kRowsPerLoad * i + lrow) * kSlots + lcol] = wl[i];
    wave_lds_sync();
#pragma unroll
    for (int u = 0; u < SG; ++u) {
      h8_t xp[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) xp[j] = pair_x8(xv[u][j]);
#pragma unroll
      for (int t = 0; t < RT; ++t) {
        const uint4 wv = wbuf[(16 * t + r_lane) * kSlots + 4 * u + kq];
        const uint32_t words[4] = {wv.x, wv.y, wv.z, wv.w};
        f4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j)
          c = __builtin_amdgcn_mfma_f32_16x16x32_f16(unpack_word_h8(words[j]), xp[j], c, 0, 0, 0);
        // A group past G loaded zero weights and scales, so it adds nothing.
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float scale = kPairs ? h2f((uint16_t)(sc2[t][v] >> (16 * u))) : sc[t][kPairs ? 0 : u][v];
          acc[t][v] = __builtin_fmaf(c[v], scale, acc[t][v]);
        }
      }
    }
    wave_lds_sync();  // the reads above complete before the next block's writes
  }
}

// LDS of the tile kernels: one staging buffer per wave. After its block
// loop (which ends with the wave's reads of the buffer complete) a wave
// stores its fp32 partials over its own buffer; after a workgroup barrier
// the summing waves read every wave's. Without a separate reduction array
// the LDS per workgroup is 31% smaller (M = K = 4096, B = 16: 6.82 against
// 7.04 us).
template <int KS, int RT, int SG>
struct ReuseLds {
  uint4 wst[KS][16 * RT * (SG * 4 + 1)];
  static_assert(sizeof(wst[0]) >= 256 * RT * sizeof(float), "partials fit a staging buffer");
};

// Adds tile t's KS wave partials in wave order (after the barrier).
template <int KS, int RT, int SG>
__device__ __forceinline__ f4_t reuse_tile_sum(const ReuseLds<KS, RT, SG>& lds, int t, int lane) {
  f4_t sum = {0.f, 0.f, 0.f, 0.f};
  for (int w2 = 0; w2 < KS; ++w2) {
    const float* part = reinterpret_cast<const float*>(lds.wst[w2]);
#pragma unroll
    for (int v = 0; v < 4; ++v) sum[v] += part[(t * 64 + lane) * 4 + v];
  }
  return sum;
}

template <int KS, int RT, int SG>
__device__ __forceinline__ void reuse_tile_publish(ReuseLds<KS, RT, SG>& lds, const f4_t (&acc)[RT],
                                                   int wave, int lane) {
  float* part = reinterpret_cast<float*>(lds.wst[wave]);
#pragma unroll
  for (int t = 0; t < RT; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) part[(t * 64 + lane) * 4 + v] = acc[t][v];
}

// GEMV: tile t of a workgroup is rows row0 + 16 t .. + 15.
template <int KS, int RT, int SG, bool kPairs>
__global__ __launch_bounds__(KS * 64) void gemv_reuse(const uint4* __restrict__ packed,
                                                      const uint16_t* __restrict__ scales,
                                                      const uint4* __restrict__ x4,
                                                      uint16_t* __restrict__ y, int M, int K,
                                                      int B) {
  static_assert(KS >= RT, "wave t sums tile t");
  __shared__ ReuseLds<KS, RT, SG> lds;
  const int G = K >> 7;
  const int nck = K >> 5;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row0 = blockIdx.x * 16 * RT;
  const int b = blockIdx.y * kReuseBatch + (lane & 15);  // this lane's batch column
  const int kq = lane >> 4;
  __amdgpu_buffer_rsrc_t rw[RT], rs[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    // A tile wholly past M gets empty descriptors: its loads read zero. The
    // row count is made wave-uniform explicitly: computed on the VALU, it
    // left the descriptors in VGPRs and every load in a readfirstlane loop
    // (M = 8192, K = 28672, B = 8: 32.8 against 46.9 us).
    const int rows = __builtin_amdgcn_readfirstlane(max(0, min(16, M - row0 - 16 * t)));
    const int rbase = rows > 0 ? row0 + 16 * t : 0;
    rw[t] = buffer_rsrc(packed + (size_t)rbase * nck, (uint32_t)(rows * (K / 2)));
    rs[t] = buffer_rsrc(scales + (size_t)rbase * G, (uint32_t)(rows * G * 2));
  }
  const auto rx = buffer_rsrc(x4, (uint32_t)((size_t)B * K * 2));
  const int xbase = b < B ? b * K * 2 + kq * 64 : kOutOfRange;
  f4_t acc[RT];
  reuse_tile_loop<KS, RT, SG, kPairs>(acc, lds.wst[wave], rw, rs, rx, xbase, G, G, nck, lane, wave,
                              b < B);
  reuse_tile_publish(lds, acc, wave, lane);
  __syncthreads();
  if (wave < RT) {
    const f4_t sum = reuse_tile_sum(lds, wave, lane);
    if (b < B) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int orow = row0 + 16 * wave + 4 * kq + v;
        if (orow < M) y[(size_t)b * M + orow] = f2h(sum[v]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Tiles with both operands staged by the buffer-load-to-LDS path (gfx950
// loads of 16 bytes per lane that write LDS directly, lane l's bytes at
// 16 l past the instruction's LDS base). The MFMA B operand takes batch row
// l % 16 in lane l, so loading it directly makes every load instruction
// touch 16 batch rows K * 2 bytes apart; at M = K = 4096, B = 16 that layout
// cost 1.8 us of 6.9 against the same bytes read in row order. Here each
// wave's block of x (16 batch rows x 512 bytes, two groups) and of weights
// (16 RT rows x 128 bytes) is read in row order, 1 KiB per instruction,
// straight into the wave's LDS, and read back in the MFMA layouts; the
// source chunk of each lane is XOR-swizzled by row so that those reads (16
// rows, one chunk) fall in 16 distinct groups of four banks with no
// padding. x loads whose batch rows are all past B are not issued. Measured
// on MI355X at M = K = 4096 (us, against gemv_reuse with the same waves and
// blocks): B = 16 5.45 (7.02), B = 12 5.10 (6.25), B = 8 4.82 (5.13), B = 4
// 4.57 (4.77). Issuing the next block before this block's wait (a second
// buffer set) gained nothing: the compiler's wait before the LDS reads also
// covers the other buffer's loads.
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void* lds_void_ptr;

// XOR applied to the chunk index of row r of a staged block with kChunks
// 16-byte chunks per row (16 rows reading one chunk hit distinct banks).
template <int kChunks>
__device__ __forceinline__ int stage_swizzle(int r) {
  if constexpr (kChunks % 16 == 0) {
    return r & 15;
  } else {
    static_assert(kChunks == 8, "rows of 8 or a multiple of 16 chunks");
    return (r >> 1) & 7;
  }
}

// Per wave, for blocks of SG groups: 16 batch rows x 16 SG chunks of x and
// 16 RT rows x 4 SG chunks of weights.
template <int KS, int RT, int SG = 2>
struct ReuseDmaLds {
  uint4 x[KS][16 * 16 * SG];
  uint4 w[KS][RT * 16 * 4 * SG];
};

// One block of SG (2 or 4) groups of the LDS-staged tiles, groups g0 ..
// g0 + SG - 1: tile t's weights and scales through descriptors rw[t], rs[t]
// (rows 0..15 relative to them, G groups per row), x of batch rows bt0 ..
// bt0 + 15 (those below B; nxl loads cover them) through rx with rows K * 2
// bytes apart, added into acc[t], this lane's part of tile t's fp32 16x16
// result. kTail: the block may run past group G - 1, so each load checks
// its group (a block that ends inside the row needs no check, and its loads
// issue with no address arithmetic beyond the loop's increments). kPairs:
// the scales of two groups in one 4-byte load (an even number of groups per
// row, 4-byte aligned).
template <int RT, bool kPairs, int SG, bool kTail>
__device__ __forceinline__ void reuse_lds_block(f4_t (&acc)[RT], uint4* xbuf, uint4* wbuf,
                                                const __amdgpu_buffer_rsrc_t (&rw)[RT],
                                                const __amdgpu_buffer_rsrc_t (&rs)[RT],
                                                __amdgpu_buffer_rsrc_t rx, int bt0, int B, int K,
                                                int G, int lane, int g0, int nxl) {
  constexpr int kWC = 4 * SG;   // weight chunks per row of a block
  constexpr int kWR = 64 / kWC;  // weight rows per load
  constexpr int kXC = 16 * SG;  // x chunks per batch row of a block
  constexpr int kXR = 64 / kXC;  // batch rows per x load
  const int nck = K >> 5;
  const int kq = lane >> 4;
  const int r_lane = lane & 15;
  // Weights: load i covers rows kWR (i % (16 / kWR)) .. + kWR - 1 of tile
  // i / (16 / kWR), lane l chunk l % kWC of row kWR (i % (16 / kWR)) + l /
  // kWC (chunk c = group c / 4 of the block, bytes 16 (c % 4) of it).
#pragma unroll
  for (int i = 0; i < RT * 16 / kWR; ++i) {
    const int r = kWR * (i % (16 / kWR)) + lane / kWC;
    const int c = (lane % kWC) ^ stage_swizzle<kWC>(r);
    const int off = !kTail || g0 * 4 + c < G * 4 ? r * nck * 16 + (g0 * 4 + c) * 16 : kOutOfRange;
    // A local copy of the descriptor: given the array element itself, the
    // host pass leaves the kernel's launch stub undefined.
    const __amdgpu_buffer_rsrc_t rwt = rw[i / (16 / kWR)];
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rwt, (lds_void_ptr)(wbuf + i * 64), 16, off, 0, 0,
                                             kLoadNonTemporal);
  }
  // Scales of this lane's four D rows: two groups in one 4-byte load where
  // the scales allow (an even number of groups, so g0 + 2v + 1 < G when
  // g0 + 2v < G).
  float sc[RT][SG][4];
#pragma unroll
  for (int t = 0; t < RT; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      if constexpr (kPairs) {
#pragma unroll
        for (int u2 = 0; u2 < SG / 2; ++u2) {
          const int g = g0 + 2 * u2;
          const uint32_t two = __builtin_amdgcn_raw_buffer_load_b32(
              rs[t], !kTail || g < G ? ((4 * kq + v) * G + g) * 2 : kOutOfRange, 0, 0);
          sc[t][2 * u2][v] = h2f((uint16_t)two);
          sc[t][2 * u2 + 1][v] = h2f((uint16_t)(two >> 16));
        }
      } else {
#pragma unroll
        for (int u = 0; u < SG; ++u) {
          const int off = !kTail || g0 + u < G ? ((4 * kq + v) * G + g0 + u) * 2 : kOutOfRange;
          sc[t][u][v] = h2f(__builtin_amdgcn_raw_buffer_load_b16(rs[t], off, 0, 0));
        }
      }
    }
  // x: load i covers batch rows bt0 + kXR i .. + kXR - 1, lane l chunk
  // l % kXC of row kXR i + l / kXC (chunk c = group c / 16, bytes 16 (c % 16)).
#pragma unroll
  for (int i = 0; i < 16 / kXR; ++i) {
    if (i < nxl) {
      const int bb = kXR * i + lane / kXC;
      const int p = lane % kXC;
      const int c = (p & ~15) | ((p ^ stage_swizzle<kXC>(bb)) & 15);
      const bool ok = bt0 + bb < B && (!kTail || g0 * 16 + c < G * 16);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rx, (lds_void_ptr)(xbuf + i * 64), 16,
          ok ? (bt0 + bb) * K * 2 + (g0 * 16 + c) * 16 : kOutOfRange, 0, 0, 0);
    }
  }
  // Every load of the block, LDS writes included, has landed.
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
  for (int u = 0; u < SG; ++u) {
    h8_t xp[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int xc = 16 * u + 4 * kq + j;
      xp[j] = pair_x8(
          xbuf[r_lane * kXC + ((xc & ~15) | ((xc ^ stage_swizzle<kXC>(r_lane)) & 15))]);
    }
#pragma unroll
    for (int t = 0; t < RT; ++t) {
      const int wc = (4 * u + kq) ^ stage_swizzle<kWC>(r_lane);
      const uint4 wv = wbuf[(16 * t + r_lane) * kWC + wc];
      const uint32_t words[4] = {wv.x, wv.y, wv.z, wv.w};
      f4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j)
        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(unpack_word_h8(words[j]), xp[j], c, 0, 0, 0);
      // A group past G loaded zero weights, so it adds nothing.
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[t][v] = __builtin_fmaf(c[v], sc[t][u][v], acc[t][v]);
    }
  }
  // The reads above have returned before the next block's loads write the
  // buffers.
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// The block loop of the LDS-staged tiles: acc[t] over the wave's blocks of
// SG groups (groups SG wave .. SG wave + SG - 1, then every SG KS), the
// blocks that end inside the row first, then the one that runs past its
// end if the row's group count is not a multiple of SG.
template <int KS, int RT, bool kPairs, int SG = 2>
__device__ __forceinline__ void reuse_lds_loop(f4_t (&acc)[RT], uint4* xbuf, uint4* wbuf,
                                               const __amdgpu_buffer_rsrc_t (&rw)[RT],
                                               const __amdgpu_buffer_rsrc_t (&rs)[RT],
                                               __amdgpu_buffer_rsrc_t rx, int bt0, int B, int K,
                                               int G, int lane, int wave) {
  static_assert(SG == 2 || SG == 4, "blocks of two or four groups");
  constexpr int kXR = 64 / (16 * SG);  // batch rows per x load
  // x loads with a batch row below B (wave-uniform).
  const int nxl = min(16 / kXR, (max(0, min(16, B - bt0)) + kXR - 1) / kXR);
#pragma unroll
  for (int t = 0; t < RT; ++t) acc[t] = f4_t{0.f, 0.f, 0.f, 0.f};
  int g0 = SG * wave;
  for (; g0 + SG <= G; g0 += SG * KS)
    reuse_lds_block<RT, kPairs, SG, false>(acc, xbuf, wbuf, rw, rs, rx, bt0, B, K, G, lane, g0,
                                           nxl);
  if (g0 < G)
    reuse_lds_block<RT, kPairs, SG, true>(acc, xbuf, wbuf, rw, rs, rx, bt0, B, K, G, lane, g0,
                                          nxl);
}

// Partials of the LDS-staged tiles over each wave's own x buffer (no other
// wave reads it before the barrier that follows), and tile t's KS partials
// added in wave order (after that barrier).
template <int KS, int RT, int SG>
__device__ __forceinline__ void reuse_lds_publish(ReuseDmaLds<KS, RT, SG>& lds,
                                                  const f4_t (&acc)[RT], int wave, int lane) {
  float* part = reinterpret_cast<float*>(lds.x[wave]);
#pragma unroll
  for (int t = 0; t < RT; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) part[(t * 64 + lane) * 4 + v] = acc[t][v];
}

template <int KS, int RT, int SG>
__device__ __forceinline__ f4_t reuse_lds_sum(const ReuseDmaLds<KS, RT, SG>& lds, int t,
                                              int lane) {
  f4_t sum = {0.f, 0.f, 0.f, 0.f};
  for (int w2 = 0; w2 < KS; ++w2) {
    const float* part = reinterpret_cast<const float*>(lds.x[w2]);
#pragma unroll
    for (int v = 0; v < 4; ++v) sum[v] += part[(t * 64 + lane) * 4 + v];
  }
  return sum;
}

template <int KS, int RT, bool kPairs, int SG = 2>
__global__ __launch_bounds__(KS * 64) void gemv_reuse_lds(const uint4* __restrict__ packed,
                                                          const uint16_t* __restrict__ scales,
                                                          const uint4* __restrict__ x4,
                                                          uint16_t* __restrict__ y, int M, int K,
                                                          int B) {
  static_assert(KS >= RT, "wave t sums tile t");
  __shared__ ReuseDmaLds<KS, RT, SG> lds;
  const int G = K >> 7;
  const int nck = K >> 5;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row0 = blockIdx.x * 16 * RT;
  const int bt0 = blockIdx.y * kReuseBatch;
  const int b = bt0 + (lane & 15);  // this lane's batch column
  const int kq = lane >> 4;
  __amdgpu_buffer_rsrc_t rw[RT], rs[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    const int rows = __builtin_amdgcn_readfirstlane(max(0, min(16, M - row0 - 16 * t)));
    const int rbase = rows > 0 ? row0 + 16 * t : 0;
    rw[t] = buffer_rsrc(packed + (size_t)rbase * nck, (uint32_t)(rows * (K / 2)));
    rs[t] = buffer_rsrc(scales + (size_t)rbase * G, (uint32_t)(rows * G * 2));
  }
  const auto rx = buffer_rsrc(x4, (uint32_t)((size_t)B * K * 2));
  f4_t acc[RT];
  reuse_lds_loop<KS, RT, kPairs, SG>(acc, lds.x[wave], lds.w[wave], rw, rs, rx, bt0, B, K, G,
                                     lane, wave);
  reuse_lds_publish(lds, acc, wave, lane);
  __syncthreads();
  if (wave < RT) {
    const f4_t sum = reuse_lds_sum(lds, wave, lane);
    if (b < B) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int orow = row0 + 16 * wave + 4 * kq + v;
        if (orow < M) y[(size_t)b * M + orow] = f2h(sum[v]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Double-buffered LDS-staged tiles: blocks of two groups with paired scales,
// block n + 1's loads issued into one buffer before block n is computed
// from the other. Per wave two buffers, each one block: 16 batch rows x 32
// chunks of x, 16 RT rows x 8 chunks of weights, and the scale pairs of
// tile t's row r in dword 64 t + r (the scale loads of lanes 16-63 land
// zeros in the rest). The scales come through LDS like the rest, so a
// block's loads write no register: the buffers reach each step as
// __restrict__ pointers, which lets the compiler wait for the block being
// computed without waiting for the one being loaded.
// ---------------------------------------------------------------------------
// XR: batch rows staged per x buffer (16, or 8 / 4 for batch tiles of at
// most that many rows; the MFMA then reads zeros for rows XR..15).
template <int KS, int RT, int XR = 16>
struct ReusePfLds {
  uint4 x[2][KS][XR * 32];
  uint4 w[2][KS][RT * 16 * 8];
  uint4 s[2][KS][RT * 16];
  int last;  // the split-K form's ticket result
  static_assert(sizeof(x[0][0]) >= 256 * RT * sizeof(float), "partials fit an x buffer");
};

// Loads per block and wave: two per tile of weights, kXL of x (two batch
// rows each), one per tile of scales.
template <int RT, int kXL>
constexpr int kReusePfLoads = 3 * RT + kXL;

// s_waitcnt vmcnt(N) alone (the gfx9 encoding, expcnt and lgkmcnt at their
// maximum).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is six bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

// Orders memory accesses for the compiler only (no instruction): the LDS
// reads after an explicit s_waitcnt must not be hoisted above it, and reads
// before an LDS-DMA issue must not sink below it. s_waitcnt and
// sched_barrier do not order memory operations before instruction
// selection; without this the compiler moved a block's weight and scale
// reads of gemv_reuse_pfb to the loop head, above the wait for their
// LDS-DMA.
__device__ __forceinline__ void compiler_fence() { asm volatile("" ::: "memory"); }

// A window of each row: groups [gbeg, gbeg + G) of a K-long row, tile t's
// weights and scales through descriptors rw[t], rs[t] (starting at group
// gbeg of the tile's first row; rows K / 2 bytes and Gs scales apart), x of
// batch rows bt0 .. bt0 + 15 (those below B) through rx (rows K * 2 bytes
// apart).
// (The descriptors travel as arrays beside it: a struct holding them is
// rejected by the host pass of a template instantiated from a kernel.)
struct ReuseWindow {
  int bt0, B, K, G, Gs, gbeg;
};

// Issues the loads of the block at window group g0 into wb, sb, xb: the
// weights and scale pairs first (from HBM), then the kXL x loads of batch
// rows bt0 .. bt0 + 2 kXL - 1 (the rows the x buffer holds; from L2), those
// of rows >= B out of range, so that each block issues the same number of
// loads. Scales before x: the block's last HBM load then starts before the
// x loads rather than after them. Against x before the scales, us (same
// inputs, the two libraries alternating): M = K = 4096, B = 8 4.47 (4.57),
// B = 16 4.92 (5.08); M = 4096, K = 11008, B = 16 9.66 (9.94); the split
// form at M = 1024, K = 28672, B = 16 14.43 (14.84); gate/up at I = 2752,
// H = 4096, B = 16 6.36 (6.74); within 1.3% at the other shapes timed.
template <int RT, int kXL>
__device__ __forceinline__ void reuse_pf_issue(uint4* __restrict__ xb, uint4* __restrict__ wb,
                                               uint4* __restrict__ sb,
                                               const __amdgpu_buffer_rsrc_t (&rw)[RT],
                                               const __amdgpu_buffer_rsrc_t (&rs)[RT],
                                               __amdgpu_buffer_rsrc_t rx, const ReuseWindow& win,
                                               int lane, int g0) {
  // Weights: load i covers rows 8 (i % 2) .. + 7 of tile i / 2, lane l
  // chunk l % 8 of row 8 (i % 2) + l / 8 (chunk c = group c / 4 of the
  // block, bytes 16 (c % 4) of it).
#pragma unroll
  for (int i = 0; i < 2 * RT; ++i) {
    const int r = 8 * (i % 2) + lane / 8;
    const int c = (lane % 8) ^ stage_swizzle<8>(r);
    const __amdgpu_buffer_rsrc_t rwt = rw[i / 2];
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rwt, (lds_void_ptr)(wb + i * 64), 16,
                                             r * (win.K / 2) + (g0 * 4 + c) * 16, 0, 0,
                                             kLoadNonTemporal);
  }
  // Scale pairs: lane r < 16 row r of tile t.
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    const __amdgpu_buffer_rsrc_t rst = rs[t];
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rst, (lds_void_ptr)(sb + 16 * t), 4,
                                             lane < 16 ? (lane * win.Gs + g0) * 2 : kOutOfRange,
                                             0, 0, 0);
  }
  // x: load i covers batch rows bt0 + 2 i, bt0 + 2 i + 1, lane l chunk
  // l % 32 of row 2 i + l / 32 (chunk c = group c / 16, bytes 16 (c % 16)).
#pragma unroll
  for (int i = 0; i < kXL; ++i) {
    const int bb = 2 * i + lane / 32;
    const int p = lane % 32;
    const int c = (p & 16) | ((p ^ stage_swizzle<32>(bb)) & 15);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rx, (lds_void_ptr)(xb + i * 64), 16,
        win.bt0 + bb < win.B ? (win.bt0 + bb) * win.K * 2 + (win.gbeg + g0) * 256 + c * 16
                             : kOutOfRange,
        0, 0, 0);
  }
}

// One step: with kNext, issues the block at gn into nx, nw, ns and waits
// for all but those loads; else waits for every load. Then adds the block
// in cx, cw, cs into acc.
template <int RT, bool kNext, int kXL>
__device__ __forceinline__ void reuse_pf_step(f4_t (&acc)[RT], const uint4* __restrict__ cx,
                                              const uint4* __restrict__ cw,
                                              const uint4* __restrict__ cs, uint4* __restrict__ nx,
                                              uint4* __restrict__ nw, uint4* __restrict__ ns,
                                              const __amdgpu_buffer_rsrc_t (&rw)[RT],
                                              const __amdgpu_buffer_rsrc_t (&rs)[RT],
                                              __amdgpu_buffer_rsrc_t rx, const ReuseWindow& win,
                                              int lane, int gn) {
  const int kq = lane >> 4;
  const int r_lane = lane & 15;
  if constexpr (kNext) {
    // The previous step's reads of the buffers about to be refilled have
    // returned (its MFMAs consumed them; this orders the loads after them).
    compiler_fence();
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_sched_barrier(0);
    reuse_pf_issue<RT, kXL>(nx, nw, ns, rw, rs, rx, win, lane, gn);
    wait_vmcnt<kReusePfLoads<RT, kXL>>();
  } else {
    wait_vmcnt<0>();
  }
  __builtin_amdgcn_sched_barrier(0);
  compiler_fence();
  uint32_t sc[RT][4];
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    const uint4 s4 = cs[16 * t + kq];  // rows 4 kq .. 4 kq + 3 of tile t
    sc[t][0] = s4.x;
    sc[t][1] = s4.y;
    sc[t][2] = s4.z;
    sc[t][3] = s4.w;
  }
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    h8_t xp[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int xc = 16 * u + 4 * kq + j;
      // Batch rows from 2 kXL on are not staged: zeros.
      const uint4 xv = 2 * kXL >= 16 || r_lane < 2 * kXL
                           ? cx[r_lane * 32 + ((xc & 16) | ((xc ^ stage_swizzle<32>(r_lane)) & 15))]
                           : uint4{0u, 0u, 0u, 0u};
      xp[j] = pair_x8(xv);
    }
#pragma unroll
    for (int t = 0; t < RT; ++t) {
      const int wc = (4 * u + kq) ^ stage_swizzle<8>(r_lane);
      const uint4 wv = cw[(16 * t + r_lane) * 8 + wc];
      const uint32_t words[4] = {wv.x, wv.y, wv.z, wv.w};
      f4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j)
        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(unpack_word_h8(words[j]), xp[j], c, 0, 0, 0);
#pragma unroll
      for (int v = 0; v < 4; ++v)
        acc[t][v] = __builtin_fmaf(c[v], h2f((uint16_t)(sc[t][v] >> (16 * u))), acc[t][v]);
    }
  }
}

// acc[t] over the wave's blocks of the window (window groups 2 wave, 2 wave
// + 1, then every 2 KS; G even), two buffers in turn; with kXL < 8 (batch
// tiles of at most 2 kXL rows) the x buffers hold 2 kXL rows.
template <int KS, int RT, int kXL = 8>
__device__ __forceinline__ void reuse_pf_loop(f4_t (&acc)[RT], ReusePfLds<KS, RT, 2 * kXL>& lds,
                                              const __amdgpu_buffer_rsrc_t (&rw)[RT],
                                              const __amdgpu_buffer_rsrc_t (&rs)[RT],
                                              __amdgpu_buffer_rsrc_t rx, const ReuseWindow& win,
                                              int lane, int wave) {
#pragma unroll
  for (int t = 0; t < RT; ++t) acc[t] = f4_t{0.f, 0.f, 0.f, 0.f};
  const int nb = max(0, (win.G / 2 - wave + KS - 1) / KS);  // blocks of this wave
  if (nb == 0) return;
  uint4* xa = lds.x[0][wave];
  uint4* xb = lds.x[1][wave];
  uint4* wa = lds.w[0][wave];
  uint4* wb = lds.w[1][wave];
  uint4* sa = lds.s[0][wave];
  uint4* sb = lds.s[1][wave];
  static_assert(kXL == 2 || kXL == 4 || kXL == 8, "x loads per block");
  int g = 2 * wave;
  reuse_pf_issue<RT, kXL>(xa, wa, sa, rw, rs, rx, win, lane, g);
  for (int n = 0;;) {
    if (n + 1 < nb) {
      reuse_pf_step<RT, true, kXL>(acc, xa, wa, sa, xb, wb, sb, rw, rs, rx, win, lane, g + 2 * KS);
    } else {
      reuse_pf_step<RT, false, kXL>(acc, xa, wa, sa, xb, wb, sb, rw, rs, rx, win, lane, 0);
      break;
    }
    ++n;
    g += 2 * KS;
    if (n + 1 < nb) {
      reuse_pf_step<RT, true, kXL>(acc, xb, wb, sb, xa, wa, sa, rw, rs, rx, win, lane, g + 2 * KS);
    } else {
      reuse_pf_step<RT, false, kXL>(acc, xb, wb, sb, xa, wa, sa, rw, rs, rx, win, lane, 0);
      break;
    }
    ++n;
    g += 2 * KS;
  }
}

// Tile t's KS wave partials, published in each wave's first x buffer (no
// other wave touches it; every load of the wave has landed) and, after a
// barrier, added in wave order.
template <int KS, int RT, int XR>
__device__ __forceinline__ void reuse_pf_publish(ReusePfLds<KS, RT, XR>& lds, const f4_t (&acc)[RT],
                                                 int wave, int lane) {
  float* part = reinterpret_cast<float*>(lds.x[0][wave]);
#pragma unroll
  for (int t = 0; t < RT; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) part[(t * 64 + lane) * 4 + v] = acc[t][v];
}

template <int KS, int RT, int XR>
__device__ __forceinline__ f4_t reuse_pf_sum(const ReusePfLds<KS, RT, XR>& lds, int t, int lane) {
  f4_t sum = {0.f, 0.f, 0.f, 0.f};
  for (int w2 = 0; w2 < KS; ++w2) {
    const float* pw = reinterpret_cast<const float*>(lds.x[0][w2]);
#pragma unroll
    for (int v = 0; v < 4; ++v) sum[v] += pw[(t * 64 + lane) * 4 + v];
  }
  return sum;
}

// Wave t < RT: tile t's sums (zeros in the other waves).
template <int KS, int RT, int XR>
__device__ __forceinline__ f4_t reuse_pf_partials(ReusePfLds<KS, RT, XR>& lds, const f4_t (&acc)[RT],
                                                  int wave, int lane) {
  reuse_pf_publish(lds, acc, wave, lane);
  __syncthreads();
  return wave < RT ? reuse_pf_sum(lds, wave, lane) : f4_t{0.f, 0.f, 0.f, 0.f};
}

// The single-pass double-buffered tiles: RT tiles of 16 rows x 16 batch
// rows per workgroup, KS waves splitting each row's blocks; kXL x loads per
// block (batch tiles of up to 2 kXL rows: B <= 2 kXL or kXL = 8). Needs an
// even number of groups per row and 4-byte aligned scales.
template <int KS, int RT, int kXL = 8>
__global__ __launch_bounds__(KS * 64) void gemv_reuse_pf(const uint4* __restrict__ packed,
                                                         const uint16_t* __restrict__ scales,
                                                         const uint4* __restrict__ x4,
                                                         uint16_t* __restrict__ y, int M, int K,
                                                         int B) {
  static_assert(KS >= RT, "wave t sums tile t");
  __shared__ ReusePfLds<KS, RT, 2 * kXL> lds;
  const int G = K >> 7;
  const int nck = K >> 5;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row0 = blockIdx.x * 16 * RT;
  __amdgpu_buffer_rsrc_t rw[RT], rs[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    const int rows = __builtin_amdgcn_readfirstlane(max(0, min(16, M - row0 - 16 * t)));
    const int rbase = rows > 0 ? row0 + 16 * t : 0;
    rw[t] = buffer_rsrc(packed + (size_t)rbase * nck, (uint32_t)(rows * (K / 2)));
    rs[t] = buffer_rsrc(scales + (size_t)rbase * G, (uint32_t)(rows * G * 2));
  }
  const auto rx = buffer_rsrc(x4, (uint32_t)((size_t)B * K * 2));
  ReuseWindow win;
  win.bt0 = blockIdx.y * kReuseBatch;
  win.B = B;
  win.K = K;
  win.G = G;
  win.Gs = G;
  win.gbeg = 0;
  f4_t acc[RT];
  reuse_pf_loop<KS, RT, kXL>(acc, lds, rw, rs, rx, win, lane, wave);
  const f4_t sum = reuse_pf_partials<KS, RT>(lds, acc, wave, lane);
  const int b = win.bt0 + (lane & 15);
  if (wave < RT && b < B) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int orow = row0 + 16 * wave + 4 * (lane >> 4) + v;
      if (orow < M) y[(size_t)b * M + orow] = f2h(sum[v]);
    }
  }
}

// ---------------------------------------------------------------------------
// The double-buffered tiles for many batch rows: a workgroup's RT 16-row
// tiles serve NBT batch tiles of 16 rows (grid.y over groups of 16 NBT batch
// rows), so each weight is loaded and decoded once per 16 NBT batch rows
// instead of once per 16, and each x load serves the RT tiles. Each wave
// decodes a block's weights once into registers (the MFMA A operands of the
// block's two halves for each tile: 8 x h8 per tile) and runs the NBT batch
// tiles' MFMAs on them, streaming x one batch tile (16 rows x 2 groups,
// 8 KiB) per step through two LDS buffers; the weights and scales of the
// next block arrive, into the other pair of buffers, during the last batch
// tile of this one. Every step issues the next step's loads before it waits
// for its own (exact vmcnt: 8 x loads, 8 + 3 RT with the next block's
// weights and scales). One grid column of NBT batch tiles replaces NBT
// columns of the single-batch-tile kernels, which repeat every weight load
// and decode per column and, with one workgroup per CU fitting in LDS, run
// the columns in rounds. NBT even; groups per row even and scales 4-byte
// aligned, as for gemv_reuse_pf.
// ---------------------------------------------------------------------------
// x of batch rows bt .. bt + 15 (those below B) for the block at group g0,
// into xb (the layout of reuse_pf_issue with kXL = 8).
__device__ __forceinline__ void reuse_pfb_issue_x(uint4* __restrict__ xb, __amdgpu_buffer_rsrc_t rx,
                                                  int bt, int B, int K, int g0, int lane) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int bb = 2 * i + lane / 32;
    const int p = lane % 32;
    const int c = (p & 16) | ((p ^ stage_swizzle<32>(bb)) & 15);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rx, (lds_void_ptr)(xb + i * 64), 16,
        bt + bb < B ? (bt + bb) * K * 2 + g0 * 256 + c * 16 : kOutOfRange, 0, 0, 0);
  }
}

// Weights and scale pairs of the block at group g0 of the RT tiles (rw[t],
// rs[t]) into wb, sb (the layout of reuse_pf_issue).
template <int RT>
__device__ __forceinline__ void reuse_pfb_issue_ws(uint4* __restrict__ wb, uint4* __restrict__ sb,
                                                   const __amdgpu_buffer_rsrc_t (&rw)[RT],
                                                   const __amdgpu_buffer_rsrc_t (&rs)[RT], int K,
                                                   int G, int g0, int lane) {
#pragma unroll
  for (int i = 0; i < 2 * RT; ++i) {
    const int r = 8 * (i % 2) + lane / 8;
    const int c = (lane % 8) ^ stage_swizzle<8>(r);
    const __amdgpu_buffer_rsrc_t rwt = rw[i / 2];
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rwt, (lds_void_ptr)(wb + i * 64), 16,
                                             r * (K / 2) + (g0 * 4 + c) * 16, 0, 0,
                                             kLoadNonTemporal);
  }
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    const __amdgpu_buffer_rsrc_t rst = rs[t];
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rst, (lds_void_ptr)(sb + 16 * t), 4,
                                             lane < 16 ? (lane * G + g0) * 2 : kOutOfRange, 0, 0,
                                             0);
  }
}

// The block's MFMA A operands (weights of tile t's row lane % 16, both halves
// of the block) and this lane's four rows' scale pairs per tile, from LDS.
template <int RT>
__device__ __forceinline__ void reuse_pfb_decode(h8_t (&a)[RT][2][4], uint32_t (&sc)[RT][4],
                                                 const uint4* __restrict__ cw,
                                                 const uint4* __restrict__ cs, int lane) {
  const int kq = lane >> 4;
  const int r_lane = lane & 15;
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    const uint4 s4 = cs[16 * t + kq];
    sc[t][0] = s4.x;
    sc[t][1] = s4.y;
    sc[t][2] = s4.z;
    sc[t][3] = s4.w;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const uint4 wv = cw[(16 * t + r_lane) * 8 + ((4 * u + kq) ^ stage_swizzle<8>(r_lane))];
      a[t][u][0] = unpack_word_h8(wv.x);
      a[t][u][1] = unpack_word_h8(wv.y);
      a[t][u][2] = unpack_word_h8(wv.z);
      a[t][u][3] = unpack_word_h8(wv.w);
    }
  }
}

// One batch tile of one block: acc[t] += tile t's products with x in cx.
template <int RT>
__device__ __forceinline__ void reuse_pfb_mma(f4_t (&acc)[RT], const h8_t (&a)[RT][2][4],
                                              const uint32_t (&sc)[RT][4],
                                              const uint4* __restrict__ cx, int lane) {
  const int kq = lane >> 4;
  const int r_lane = lane & 15;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    h8_t xp[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int xc = 16 * u + 4 * kq + j;
      xp[j] = pair_x8(cx[r_lane * 32 + ((xc & 16) | ((xc ^ stage_swizzle<32>(r_lane)) & 15))]);
    }
#pragma unroll
    for (int t = 0; t < RT; ++t) {
      f4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j)
        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[t][u][j], xp[j], c, 0, 0, 0);
#pragma unroll
      for (int v = 0; v < 4; ++v)
        acc[t][v] = __builtin_fmaf(c[v], h2f((uint16_t)(sc[t][v] >> (16 * u))), acc[t][v]);
    }
  }
}

// One block of NBT steps: weights and scales in cw, cs; batch tile 0's x in
// xa, then alternately xb, xa, ... With kNext the last step issues the next
// block (group gn) into nw, ns and its tile 0 into xa.
template <int RT, int NBT, bool kNext>
__device__ __forceinline__ void reuse_pfb_block(f4_t (&acc)[NBT][RT], const uint4* __restrict__ cw,
                                                const uint4* __restrict__ cs,
                                                uint4* __restrict__ nw, uint4* __restrict__ ns,
                                                uint4* __restrict__ xa, uint4* __restrict__ xb,
                                                const __amdgpu_buffer_rsrc_t (&rw)[RT],
                                                const __amdgpu_buffer_rsrc_t (&rs)[RT],
                                                __amdgpu_buffer_rsrc_t rx, int bt0, int B, int K,
                                                int G, int g, int gn, int lane) {
  static_assert(NBT % 2 == 0, "steps alternate between two x buffers within a block");
  h8_t a[RT][2][4];
  uint32_t sc[RT][4];
#pragma unroll
  for (int t = 0; t < NBT; t += 2) {
    // Step t: x in xa; issue batch tile t + 1 into xb.
    compiler_fence();
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): earlier reads of xb have returned
    __builtin_amdgcn_sched_barrier(0);
    reuse_pfb_issue_x(xb, rx, bt0 + 16 * (t + 1), B, K, g, lane);
    wait_vmcnt<8>();
    __builtin_amdgcn_sched_barrier(0);
    compiler_fence();
    if (t == 0) reuse_pfb_decode<RT>(a, sc, cw, cs, lane);
    reuse_pfb_mma<RT>(acc[t], a, sc, xa, lane);
    // Step t + 1: x in xb; issue tile t + 2 into xa, or the next block.
    compiler_fence();
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_sched_barrier(0);
    if (t + 2 < NBT) {
      reuse_pfb_issue_x(xa, rx, bt0 + 16 * (t + 2), B, K, g, lane);
      wait_vmcnt<8>();
    } else if constexpr (kNext) {
      reuse_pfb_issue_ws<RT>(nw, ns, rw, rs, K, G, gn, lane);
      reuse_pfb_issue_x(xa, rx, bt0, B, K, gn, lane);
      wait_vmcnt<8 + 3 * RT>();
    } else {
      wait_vmcnt<0>();
    }
    __builtin_amdgcn_sched_barrier(0);
    compiler_fence();
    reuse_pfb_mma<RT>(acc[t + 1], a, sc, xb, lane);
  }
}

template <int KS, int RT, int NBT>
__global__ __launch_bounds__(KS * 64) void gemv_reuse_pfb(const uint4* __restrict__ packed,
                                                          const uint16_t* __restrict__ scales,
                                                          const uint4* __restrict__ x4,
                                                          uint16_t* __restrict__ y, int M, int K,
                                                          int B) {
  static_assert(NBT * RT <= 16, "the partials fit a wave's two x buffers");
  __shared__ ReusePfLds<KS, RT, 16> lds;
  const int G = K >> 7;
  const int nck = K >> 5;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row0 = blockIdx.x * 16 * RT;
  const int bt0 = blockIdx.y * 16 * NBT;
  __amdgpu_buffer_rsrc_t rw[RT], rs[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    const int rows = __builtin_amdgcn_readfirstlane(max(0, min(16, M - row0 - 16 * t)));
    const int rbase = rows > 0 ? row0 + 16 * t : 0;
    rw[t] = buffer_rsrc(packed + (size_t)rbase * nck, (uint32_t)(rows * (K / 2)));
    rs[t] = buffer_rsrc(scales + (size_t)rbase * G, (uint32_t)(rows * G * 2));
  }
  const auto rx = buffer_rsrc(x4, (uint32_t)((size_t)B * K * 2));
  f4_t acc[NBT][RT];
#pragma unroll
  for (int b = 0; b < NBT; ++b)
#pragma unroll
    for (int t = 0; t < RT; ++t) acc[b][t] = f4_t{0.f, 0.f, 0.f, 0.f};
  // This wave's blocks: window groups 2 wave, then every 2 KS.
  const int nb = max(0, (G / 2 - wave + KS - 1) / KS);
  if (nb > 0) {
    uint4* xa = lds.x[0][wave];
    uint4* xb = lds.x[1][wave];
    uint4* wa = lds.w[0][wave];
    uint4* wb = lds.w[1][wave];
    uint4* sa = lds.s[0][wave];
    uint4* sb = lds.s[1][wave];
    int g = 2 * wave;
    reuse_pfb_issue_ws<RT>(wa, sa, rw, rs, K, G, g, lane);
    reuse_pfb_issue_x(xa, rx, bt0, B, K, g, lane);
    for (int n = 0;;) {
      if (n + 1 < nb) {
        reuse_pfb_block<RT, NBT, true>(acc, wa, sa, wb, sb, xa, xb, rw, rs, rx, bt0, B, K, G, g,
                                       g + 2 * KS, lane);
      } else {
        reuse_pfb_block<RT, NBT, false>(acc, wa, sa, wb, sb, xa, xb, rw, rs, rx, bt0, B, K, G, g,
                                        0, lane);
        break;
      }
      ++n;
      g += 2 * KS;
      if (n + 1 < nb) {
        reuse_pfb_block<RT, NBT, true>(acc, wb, sb, wa, sa, xa, xb, rw, rs, rx, bt0, B, K, G, g,
                                       g + 2 * KS, lane);
      } else {
        reuse_pfb_block<RT, NBT, false>(acc, wb, sb, wa, sa, xa, xb, rw, rs, rx, bt0, B, K, G, g,
                                        0, lane);
        break;
      }
      ++n;
      g += 2 * KS;
    }
  }
  // Every load of this wave has landed (the last step waited for all). Each
  // wave's partials of (batch tile b, row tile t), i = b RT + t, go to its x
  // buffer i / 8, slot i % 8; after the barrier wave w adds items w, w + KS,
  // ... over the KS waves in wave order.
  compiler_fence();
#pragma unroll
  for (int b = 0; b < NBT; ++b)
#pragma unroll
    for (int t = 0; t < RT; ++t) {
      const int i = b * RT + t;
      float* part = reinterpret_cast<float*>(lds.x[i / 8][wave]) + (i % 8) * 256;
#pragma unroll
      for (int v = 0; v < 4; ++v) part[lane * 4 + v] = acc[b][t][v];
    }
  __syncthreads();
  const int kq = lane >> 4;
  for (int i = wave; i < NBT * RT; i += KS) {
    f4_t sum = {0.f, 0.f, 0.f, 0.f};
    for (int w2 = 0; w2 < KS; ++w2) {
      const float* part = reinterpret_cast<const float*>(lds.x[i / 8][w2]) + (i % 8) * 256;
#pragma unroll
      for (int v = 0; v < 4; ++v) sum[v] += part[lane * 4 + v];
    }
    const int bcol = bt0 + 16 * (i / RT) + (lane & 15);
    if (bcol < B) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int orow = row0 + 16 * (i % RT) + 4 * kq + v;
        if (orow < M) y[(size_t)bcol * M + orow] = f2h(sum[v]);
      }
    }
  }
}

// The end of a split-K tile workgroup (blockIdx.z = slice z of gridDim.z):
// wave t < RT holds tile t's sums over the slice for its lane's four rows
// and batch column b in sum. Writes them to partials[z][b][row]
// (agent-scope stores, past the non-coherent L2s) and takes a ticket; the
// last of the slices to arrive adds them in order z = 0, 1, ...
// (bit-reproducible) and writes y.
template <int RT>
__device__ __forceinline__ void reuse_split_finish(const f4_t& sum, int& last,
                                                   uint16_t* __restrict__ y,
                                                   float* __restrict__ partials,
                                                   unsigned long long* __restrict__ tickets,
                                                   unsigned long long gen, int row0, int b, int M,
                                                   int B, int wave, int lane) {
  const int S = gridDim.z;
  const int split = blockIdx.z;
  const int kq = lane >> 4;
  if (wave < RT && b < B) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int orow = row0 + 16 * wave + 4 * kq + v;
      if (orow < M)
        __hip_atomic_store(&partials[((size_t)split * B + b) * M + orow], sum[v], __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  // Every wave's partial stores are complete before the ticket is taken.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  unsigned long long* ticket = &tickets[blockIdx.y * gridDim.x + blockIdx.x];
  if (threadIdx.x == 0) last = take_ticket(ticket, gen, S);
  __syncthreads();
  if (!last) return;
  if (wave < RT && b < B) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int orow = row0 + 16 * wave + 4 * kq + v;
      if (orow >= M) continue;
      float total = 0.f;
      for (int z = 0; z < S; ++z)
        total += __hip_atomic_load(&partials[((size_t)z * B + b) * M + orow], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
      y[(size_t)b * M + orow] = f2h(total);
    }
  }
  if (threadIdx.x == 0) release_ticket(ticket, gen);
}

// Split-K form for rows too few to give every CU a tile with the whole row:
// grid.z = S workgroups share each set of RT tiles, workgroup z covering
// groups [z * ceil(G / S), +ceil(G / S)), so each reads only its slice of
// the activations. Each writes its fp32 tile sums to partials[z][b][row]
// (agent-scope stores, past the non-coherent L2s) and takes a ticket; the
// last of the S adds the slices in order z = 0..S-1 (bit-reproducible) and
// writes y. The tickets are those of the v4 split-K (take_ticket): a
// workspace needs no clearing.
template <int KS, int RT, int SG>
__global__ __launch_bounds__(KS * 64) void gemv_reuse_split(
    const uint4* __restrict__ packed, const uint16_t* __restrict__ scales,
    const uint4* __restrict__ x4, uint16_t* __restrict__ y, float* __restrict__ partials,
    unsigned long long* __restrict__ tickets, unsigned long long gen, int M, int K, int B) {
  static_assert(KS >= RT, "wave t sums tile t");
  __shared__ ReuseLds<KS, RT, SG> lds;
  __shared__ int last;
  const int S = gridDim.z;
  const int split = blockIdx.z;
  const int Gall = K >> 7;
  const int gps = (Gall + S - 1) / S;
  const int gbeg = min(split * gps, Gall);
  const int G = min(gbeg + gps, Gall) - gbeg;  // groups of this slice (0 if none)
  const int nck = K >> 5;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row0 = blockIdx.x * 16 * RT;
  const int b = blockIdx.y * kReuseBatch + (lane & 15);  // this lane's batch column
  const int kq = lane >> 4;
  __amdgpu_buffer_rsrc_t rw[RT], rs[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    // Descriptors start at the slice's first group of the tile's first row
    // and end after its last group of the tile's last row.
    const int rows = max(0, min(16, M - row0 - 16 * t));
    const int rbase = rows > 0 ? row0 + 16 * t : 0;
    const uint32_t wbytes = rows > 0 ? (uint32_t)((rows - 1) * (K / 2) + G * 64) : 0u;
    const uint32_t sbytes = rows > 0 ? (uint32_t)(((rows - 1) * Gall + G) * 2) : 0u;
    rw[t] = buffer_rsrc(packed + (size_t)rbase * nck + (size_t)gbeg * 4, wbytes);
    rs[t] = buffer_rsrc(scales + (size_t)rbase * Gall + gbeg, sbytes);
  }
  const auto rx = buffer_rsrc(x4, (uint32_t)((size_t)B * K * 2));
  const int xbase = b < B ? b * K * 2 + gbeg * 256 + kq * 64 : kOutOfRange;
  f4_t acc[RT];
  reuse_tile_loop<KS, RT, SG>(acc, lds.wst[wave], rw, rs, rx, xbase, G, Gall, nck, lane, wave,
                              b < B);
  reuse_tile_publish(lds, acc, wave, lane);
  __syncthreads();
  f4_t sum = {0.f, 0.f, 0.f, 0.f};
  if (wave < RT) sum = reuse_tile_sum(lds, wave, lane);
  reuse_split_finish<RT>(sum, last, y, partials, tickets, gen, row0, b, M, B, wave, lane);
}

// The double-buffered tiles in split-K form: grid.z = S workgroups share
// each set of RT tiles, workgroup z covering groups [z gps, (z + 1) gps) of
// every row, gps = 2 ceil(G / 2S) (whole blocks of two groups), then
// reuse_split_finish. Needs an even number of groups per row and 4-byte
// aligned scales.
template <int KS, int RT>
__global__ __launch_bounds__(KS * 64) void gemv_reuse_split_pf(
    const uint4* __restrict__ packed, const uint16_t* __restrict__ scales,
    const uint4* __restrict__ x4, uint16_t* __restrict__ y, float* __restrict__ partials,
    unsigned long long* __restrict__ tickets, unsigned long long gen, int M, int K, int B) {
  static_assert(KS >= RT, "wave t sums tile t");
  __shared__ ReusePfLds<KS, RT> lds;
  const int S = gridDim.z;
  const int Gall = K >> 7;
  const int gps = 2 * ((Gall + 2 * S - 1) / (2 * S));
  const int gbeg = min((int)blockIdx.z * gps, Gall);
  const int G = min(gbeg + gps, Gall) - gbeg;  // groups of this slice (even; 0 if none)
  const int nck = K >> 5;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row0 = blockIdx.x * 16 * RT;
  __amdgpu_buffer_rsrc_t rw[RT], rs[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    // Descriptors start at the slice's first group of the tile's first row
    // and end after its last group of the tile's last row.
    const int rows = __builtin_amdgcn_readfirstlane(max(0, min(16, M - row0 - 16 * t)));
    const int rbase = rows > 0 ? row0 + 16 * t : 0;
    const uint32_t wbytes = rows > 0 ? (uint32_t)((rows - 1) * (K / 2) + G * 64) : 0u;
    const uint32_t sbytes = rows > 0 ? (uint32_t)(((rows - 1) * Gall + G) * 2) : 0u;
    rw[t] = buffer_rsrc(packed + (size_t)rbase * nck + (size_t)gbeg * 4, wbytes);
    rs[t] = buffer_rsrc(scales + (size_t)rbase * Gall + gbeg, sbytes);
  }
  const auto rx = buffer_rsrc(x4, (uint32_t)((size_t)B * K * 2));
  ReuseWindow win;
  win.bt0 = blockIdx.y * kReuseBatch;
  win.B = B;
  win.K = K;
  win.G = G;
  win.Gs = Gall;
  win.gbeg = gbeg;
  f4_t acc[RT];
  reuse_pf_loop<KS, RT>(acc, lds, rw, rs, rx, win, lane, wave);
  const f4_t sum = reuse_pf_partials<KS, RT>(lds, acc, wave, lane);
  reuse_split_finish<RT>(sum, lds.last, y, partials, tickets, gen, row0, win.bt0 + (lane & 15), M,
                         B, wave, lane);
}

}  // namespace dk
