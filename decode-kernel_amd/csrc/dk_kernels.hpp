// Every W4A16 GEMV kernel for gfx950, as templates and __global__ functions.
// Included by exactly one translation unit of the library (dk_gemv.hip),
// which owns the one __device__ global defined here (the dispatch stamp).
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
// Dispatch stamp: written by block (0,0) thread 0 of whichever GEMV kernel
// ran. Host reads and clears it in dk_last_kernel_stamp().
// Reference: csrc/gemv_w4a16.cu:18-25.
// ---------------------------------------------------------------------------
__device__ int g_stamp = -1;

__device__ __forceinline__ void write_stamp(int s) {
  if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) g_stamp = s;
}

// ---------------------------------------------------------------------------
// v0: one thread per row, scalar decode (the uncoalesced baseline stage).
// Reference: csrc/gemv_w4a16.cu:70-94.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void gemv_v0(const uint32_t* __restrict__ packed,
                                               const uint16_t* __restrict__ scales,
                                               const uint16_t* __restrict__ x,
                                               uint16_t* __restrict__ y, int M, int K, int B) {
  write_stamp(0);
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
  write_stamp(1);
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
  write_stamp(10 + wpr);
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
  write_stamp(kScalesInLds ? 3 : 2);
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
// v5: the tuned streaming kernel. Each wave owns R consecutive rows; lane l
// owns 16-byte chunks l, l+64, ... of each of them, U chunks per lane per
// stage. All loads of a stage are raw buffer loads through SGPR resource
// descriptors scoped to the wave's rows (a chunk past the row end, or a row
// past M, is an out-of-range offset that reads 0, so tails need no branches
// and the loads issue back to back): the NB activation chunks first, then
// the scales, then the weights with the non-temporal hint (read-once data).
// Activations are paired once per stage and reused for all R rows. Load
// latency is hidden by the other waves on the SIMD, not by double buffering
// inside a wave (2% slower at M = K = 4096 and 20% at M = 4096, K = 11008
// once the decode was 13 ops per word).
// grid.y covers the batch in tiles of NB rows; workgroup ids are renumbered
// so each XCD streams one contiguous block of rows (measured 2-5% faster).
// Reference: csrc/gemv_w4a16.cu:318-357.
// ---------------------------------------------------------------------------
constexpr int kOutOfRange = (int)0x80000000;  // beyond any descriptor's num_records
// Waves per workgroup of the streaming kernels (v5 and the fused gate/up):
// a compile-time constant, so no wave reads the dispatch packet's workgroup
// size before issuing its first load.
constexpr int kStreamWaves = 2;
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

template <int R, int U, int NB>
struct V5Stage {
  uint4 w[U][R];
  float s[U][R];
  uint4 xv[U][NB][4];
};

// Loads one stage: rows r < kSplit come from (rw, rs), rows r >= kSplit
// from (rw2, rs2) as their row r - kSplit (the fused gate/up kernel streams
// two matrices against one activation load; plain v5 has kSplit = R).
template <int R, int U, int NB, int kSplit = R>
__device__ __forceinline__ void v5_load(V5Stage<R, U, NB>& st, __amdgpu_buffer_rsrc_t rw,
                                        __amdgpu_buffer_rsrc_t rs, __amdgpu_buffer_rsrc_t rx,
                                        int c0, int nck, int G, int K, int b0, int B, int lane,
                                        __amdgpu_buffer_rsrc_t rw2, __amdgpu_buffer_rsrc_t rs2) {
  int c[U];
  bool ok[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    c[u] = c0 + u * kWave + lane;
    ok[u] = c[u] < nck;
  }
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int off = (ok[u] && b0 + b < B) ? (b0 + b) * K * 2 + c[u] * 64 : kOutOfRange;
#pragma unroll
      for (int j = 0; j < 4; ++j) st.xv[u][b][j] = buffer_load16<0>(rx, off + 16 * j);
    }
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int rr = r < kSplit ? r : r - kSplit;
      const int off = ok[u] ? (rr * G + (c[u] >> 2)) * 2 : kOutOfRange;
      st.s[u][r] = h2f(__builtin_amdgcn_raw_buffer_load_b16(r < kSplit ? rs : rs2, off, 0, 0));
    }
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int rr = r < kSplit ? r : r - kSplit;
      const int off = ok[u] ? (rr * nck + c[u]) * 16 : kOutOfRange;
      st.w[u][r] = buffer_load16<kLoadNonTemporal>(r < kSplit ? rw : rw2, off);
    }
}

template <int R, int U, int NB>
__device__ __forceinline__ void v5_load(V5Stage<R, U, NB>& st, __amdgpu_buffer_rsrc_t rw,
                                        __amdgpu_buffer_rsrc_t rs, __amdgpu_buffer_rsrc_t rx,
                                        int c0, int nck, int G, int K, int b0, int B, int lane) {
  v5_load<R, U, NB, R>(st, rw, rs, rx, c0, nck, G, K, b0, B, lane, rw, rs);
}

template <int R, int U, int NB, typename Layout = LayoutLogical>
__device__ __forceinline__ void v5_compute(const V5Stage<R, U, NB>& st, float (&acc)[NB][R]) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    h2_t xp[NB][4][4];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int j = 0; j < 4; ++j) Layout::pair(st.xv[u][b][j], xp[b][j]);
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
#pragma unroll
      for (int b = 0; b < NB; ++b) acc[b][r] = __builtin_fmaf(part[b], st.s[u][r], acc[b][r]);
    }
  }
}

// kStamp is the layout's stamp, or the reuse path's when that path runs this
// kernel for one or two batch rows.
template <int R, int U, int NB, typename Layout = LayoutLogical, int kStamp = Layout::kStamp>
__global__ __launch_bounds__(kStreamWaves * 64) void gemv_v5(const uint4* __restrict__ packed,
                                                             const uint16_t* __restrict__ scales,
                                                             const uint4* __restrict__ x4,
                                                             uint16_t* __restrict__ y, int M, int K,
                                                             int B) {
  write_stamp(kStamp);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // The grid size follows from M (it is the launch's), so no hidden argument
  // is read before the first load.
  const int wg = xcd_contiguous_block(blockIdx.x, (M + kStreamWaves * R - 1) / (kStreamWaves * R));
  const int row0 = (wg * kStreamWaves + wave) * R;
  if (row0 >= M) return;  // wave-uniform; no barriers in this kernel
  const int b0 = blockIdx.y * NB;
  const int nck = K >> 5;
  const int G = K >> 7;
  const int rows = min(R, M - row0);
  // Descriptors cover only this wave's rows and the activations: every valid
  // offset stays below 2^31 and rows past M read as zero.
  const auto rw = buffer_rsrc(packed + (size_t)row0 * nck, (uint32_t)(rows * (K / 2)));
  const auto rs = buffer_rsrc(scales + (size_t)row0 * G, (uint32_t)(rows * G * 2));
  const auto rx = buffer_rsrc(x4, (uint32_t)((size_t)B * K * 2));

  float acc[NB][R];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[b][r] = 0.f;

  constexpr int kStep = U * kWave;
  V5Stage<R, U, NB> st;
  for (int c0 = 0; c0 < nck; c0 += kStep) {
    v5_load(st, rw, rs, rx, c0, nck, G, K, b0, B, lane);
    // With the paired layout's shorter math the scheduler interleaves it
    // between the stage's loads, which cuts the loads in flight per wave (it
    // made that layout 23% slower at M = 8192, K = 28672); the barrier keeps
    // them back to back. For the logical layout it changes nothing beyond
    // +-2%, so it is a trait of the layout.
    if constexpr (Layout::kLoadsFirst) __builtin_amdgcn_sched_barrier(0);
    v5_compute<R, U, NB, Layout>(st, acc);
  }

#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float t = wave_sum(acc[b][r]);
      if (lane == 63 && row0 + r < M && b0 + b < B) y[(size_t)(b0 + b) * M + row0 + r] = f2h(t);
    }
}

// ---------------------------------------------------------------------------
// v5 for one activation row, with the activations shared through LDS (stamp 5,
// or the layout's). A workgroup of W waves streams R rows per wave as gemv_v5
// does, but each stage's activations (U * 4 KiB) are loaded once per
// workgroup, one or two 16-byte loads per lane, paired once, and read by
// every wave from LDS. gemv_v5 re-reads them per wave from L2, twice the
// weight bytes at two rows per wave; that traffic and the pairing were the
// largest cost left beside the weights (4-21% at the shapes measured).
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
// ---------------------------------------------------------------------------
template <int R, int U, int W>
struct LdsStage {
  static constexpr int kPieces = U * 4 * kWave;  // 16-byte activation pieces per stage
  static constexpr int kPer = (kPieces + W * kWave - 1) / (W * kWave);
  uint4 xv[kPer];
  uint4 w[U][R];
  uint32_t s[U][R];  // raw fp16 scale bits, converted where used
};

template <int R, int U, int W>
__device__ __forceinline__ void lds_stage_load(LdsStage<R, U, W>& st, __amdgpu_buffer_rsrc_t rw,
                                               __amdgpu_buffer_rsrc_t rs, __amdgpu_buffer_rsrc_t rx,
                                               int c0, int nck, int G, int tid, int lane) {
  using S = LdsStage<R, U, W>;
  // Activations of chunks [c0, c0 + 64U): piece p is bytes [16p, 16p + 16)
  // of that range, so consecutive lanes read consecutive 16 bytes.
#pragma unroll
  for (int i = 0; i < S::kPer; ++i) {
    const int piece = tid + i * W * kWave;
    const int c = c0 + (piece >> 2);
    st.xv[i] = buffer_load16<0>(
        rx, (piece < S::kPieces && c < nck) ? (c0 * 4 + piece) * 16 : kOutOfRange);
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int c = c0 + u * kWave + lane;
    const bool ok = c < nck;
#pragma unroll
    for (int r = 0; r < R; ++r)
      st.s[u][r] = __builtin_amdgcn_raw_buffer_load_b16(rs, ok ? (r * G + (c >> 2)) * 2 : kOutOfRange,
                                                        0, 0);
#pragma unroll
    for (int r = 0; r < R; ++r)
      st.w[u][r] = buffer_load16<kLoadNonTemporal>(rw, ok ? (r * nck + c) * 16 : kOutOfRange);
  }
}

// Pairs this lane's activation pieces for the layout and stores them where
// the lane that owns the chunk reads them: xs[u][j][l] holds the four pairs
// of bytes [16j, 16j + 16) of chunk c0 + 64u + l.
template <int R, int U, int W, typename Layout>
__device__ __forceinline__ void lds_stage_publish(const LdsStage<R, U, W>& st,
                                                  uint4 (&xs)[U][4][kWave], int tid) {
  using S = LdsStage<R, U, W>;
#pragma unroll
  for (int i = 0; i < S::kPer; ++i) {
    const int piece = tid + i * W * kWave;
    if (S::kPieces % (W * kWave) == 0 || piece < S::kPieces) {
      h2_t p[4];
      Layout::pair(st.xv[i], p);
      const int cr = piece >> 2;
      xs[cr / kWave][piece & 3][cr % kWave] =
          make_uint4(__builtin_bit_cast(uint32_t, p[0]), __builtin_bit_cast(uint32_t, p[1]),
                     __builtin_bit_cast(uint32_t, p[2]), __builtin_bit_cast(uint32_t, p[3]));
    }
  }
}

template <int R, int U, int W, typename Layout>
__device__ __forceinline__ void lds_stage_compute(const LdsStage<R, U, W>& st,
                                                  const uint4 (&xs)[U][4][kWave], float (&acc)[R],
                                                  int lane) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    h2_t xp[4][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint4 pv = xs[u][j][lane];
      xp[j][0] = as_h2(pv.x);
      xp[j][1] = as_h2(pv.y);
      xp[j][2] = as_h2(pv.z);
      xp[j][3] = as_h2(pv.w);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t words[4] = {st.w[u][r].x, st.w[u][r].y, st.w[u][r].z, st.w[u][r].w};
      float part = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        h2_t q[4];
        Layout::unpack(words[j], q);
        part = __builtin_amdgcn_fdot2(q[0], xp[j][0], part, false);
        part = __builtin_amdgcn_fdot2(q[1], xp[j][1], part, false);
        part = __builtin_amdgcn_fdot2(q[2], xp[j][2], part, false);
        part = __builtin_amdgcn_fdot2(q[3], xp[j][3], part, false);
      }
      acc[r] = __builtin_fmaf(part, h2f((uint16_t)st.s[u][r]), acc[r]);
    }
  }
}

template <int R, int U, int W, bool kPrefetch, typename Layout = LayoutLogical,
          int kStamp = Layout::kStamp>
__global__ __launch_bounds__(W * kWave) void gemv_v5_lds(const uint4* __restrict__ packed,
                                                         const uint16_t* __restrict__ scales,
                                                         const uint4* __restrict__ x4,
                                                         uint16_t* __restrict__ y, int M, int K) {
  write_stamp(kStamp);
  __shared__ uint4 xs[2][U][4][kWave];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wg = xcd_contiguous_block(blockIdx.x, (M + W * R - 1) / (W * R));
  const int row0 = (wg * W + wave) * R;
  const bool active = row0 < M;  // wave-uniform
  const int nck = K >> 5;
  const int G = K >> 7;
  // An inactive wave gets empty weight and scale descriptors: all its
  // weight and scale loads read zero.
  const int rows = active ? min(R, M - row0) : 0;
  const int rbase = active ? row0 : 0;
  const auto rw = buffer_rsrc(packed + (size_t)rbase * nck, (uint32_t)(rows * (K / 2)));
  const auto rs = buffer_rsrc(scales + (size_t)rbase * G, (uint32_t)(rows * G * 2));
  const auto rx = buffer_rsrc(x4, (uint32_t)K * 2);

  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
  constexpr int kStep = U * kWave;
  if constexpr (kPrefetch) {
    LdsStage<R, U, W> sa, sb;
    lds_stage_load(sa, rw, rs, rx, 0, nck, G, tid, lane);
    for (int c0 = 0;;) {
      lds_stage_publish<R, U, W, Layout>(sa, xs[0], tid);
      __syncthreads();
      lds_stage_load(sb, rw, rs, rx, c0 + kStep, nck, G, tid, lane);
      __builtin_amdgcn_sched_barrier(0);
      lds_stage_compute<R, U, W, Layout>(sa, xs[0], acc, lane);
      c0 += kStep;
      if (c0 >= nck) break;
      lds_stage_publish<R, U, W, Layout>(sb, xs[1], tid);
      __syncthreads();
      lds_stage_load(sa, rw, rs, rx, c0 + kStep, nck, G, tid, lane);
      __builtin_amdgcn_sched_barrier(0);
      lds_stage_compute<R, U, W, Layout>(sb, xs[1], acc, lane);
      c0 += kStep;
      if (c0 >= nck) break;
    }
  } else {
    LdsStage<R, U, W> st;
    int buf = 0;
    for (int c0 = 0; c0 < nck; c0 += kStep, buf ^= 1) {
      lds_stage_load(st, rw, rs, rx, c0, nck, G, tid, lane);
      lds_stage_publish<R, U, W, Layout>(st, xs[buf], tid);
      __syncthreads();
      lds_stage_compute<R, U, W, Layout>(st, xs[buf], acc, lane);
    }
  }
  if (!active) return;  // after the last barrier
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float t = wave_sum(acc[r]);
    if (lane == 63 && row0 + r < M) y[row0 + r] = f2h(t);
  }
}

// ---------------------------------------------------------------------------
// v4: split-K. grid = (row tiles of 4, S). Workgroup (tile, s) computes the
// fp32 partial of its 4 rows over group slice s and stores it to
// ws[s][b][row]; the last workgroup of a tile to finish adds the S partials
// in slice order and writes fp16 y. One launch, deterministic.
// Reference: csrc/gemv_w4a16.cu:264-313, 415-419 (memset + atomics + convert).
//
// The completion tickets (one uint32 per tile) live in the caller's
// workspace after the partials, so launches on different streams with their
// own workspaces never share them. They must be zero when a launch starts;
// the last workgroup of each tile resets its ticket, so a workspace that was
// zeroed once stays valid for every later launch that uses it in turn.
//
// Cross-workgroup visibility on an 8-XCD part (one L2 per XCD, not coherent
// with each other) uses agent-scope atomic stores and loads for the partials
// (they bypass the non-coherent L2s) and a wait for their completion before
// the ticket, instead of agent-scope fences: a fence writes back and
// invalidates a whole L2 per wave and made this kernel ~35x slower.
// ---------------------------------------------------------------------------
constexpr int kV4TileRows = 4;  // rows per workgroup and ticket tile: one wave per row

__global__ __launch_bounds__(256) void gemv_v4(const uint4* __restrict__ packed,
                                               const uint16_t* __restrict__ scales,
                                               const uint4* __restrict__ x4,
                                               uint16_t* __restrict__ y, float* __restrict__ ws,
                                               unsigned int* __restrict__ tickets, int M, int K,
                                               int B) {
  write_stamp(4);
  __shared__ int last;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int rows_per_tile = kV4TileRows;
  const int tile = blockIdx.x;
  const int row_raw = tile * rows_per_tile + wave;
  const int row = row_raw < M ? row_raw : M - 1;
  const int S = gridDim.y;
  const int split = blockIdx.y;
  const int G = K >> 7;
  const int gps = (G + S - 1) / S;
  const int g0 = min(split * gps, G);
  const int g1 = min(g0 + gps, G);
  const int nck = K >> 5;
  const uint4* rw = packed + (size_t)row * nck;
  const uint16_t* rs = scales + (size_t)row * G;

  for (int b = 0; b < B; ++b) {
    const uint4* xb = x4 + (size_t)b * (K >> 3);
    float acc = 0.f;
    for (int c = 4 * g0 + lane; c < 4 * g1; c += kWave) {
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
      acc += h2f(rs[c >> 2]) * part;
    }
    acc = wave_sum(acc);
    if (lane == 63 && row_raw < M)
      __hip_atomic_store(&ws[((size_t)split * B + b) * M + row], acc, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }

  // Every wave's partial stores are complete before the ticket is taken.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned prev =
        __hip_atomic_fetch_add(&tickets[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = (prev == (unsigned)(S - 1));
  }
  __syncthreads();
  if (!last) return;
  const int row_base = tile * rows_per_tile;
  const int n_out = rows_per_tile * B;
  for (int t = threadIdx.x; t < n_out; t += blockDim.x) {
    const int r = row_base + (t % rows_per_tile);
    const int b = t / rows_per_tile;
    if (r >= M) continue;
    float sum = 0.f;
    for (int s = 0; s < S; ++s)
      sum += __hip_atomic_load(&ws[((size_t)s * B + b) * M + r], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    y[(size_t)b * M + r] = f2h(sum);
  }
  if (threadIdx.x == 0)
    __hip_atomic_store(&tickets[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Weight-reuse path (stamp 15): each decoded weight is used for up to 16
// batch rows at once by v_mfma_f32_16x16x32_f16, so latency is nearly flat
// in B instead of the reference's O(B) re-decode (csrc/gemv_w4a16.cu:364-413).
// A workgroup of KS waves owns one 16-row tile; wave w takes groups w, w+KS,
// ... (adjacent groups stream side by side). Lane l loads row l%16, bytes
// [64g + 16(l/16), +16) of group g: four words = four MFMA k-steps that
// together cover exactly group g, so the fp32 tile result of a group is
// scaled once and accumulated. The KS wave partials are added in LDS in wave
// order. Loads are raw buffer loads; rows past M and batch rows past B read
// zero through out-of-range offsets.
//   A (16x32, weights): lane l -> row l%16, 8 k-slots of lane group l/16
//   B (32x16, x):       lane l -> batch l%16, same 8 k-slots
//   D (16x16):          lane l -> rows 4(l/16)+v, batch l%16
// Scales, two ways (kStaged):
//   * staged: the tile's scales are copied transposed into LDS first, then
//     one group per iteration (best for long rows, where the copy is
//     amortised over many groups);
//   * direct: no staging round trip before the first weight load; each lane
//     loads the four scales of its D rows with the activations and weights,
//     UG groups per stage (best for K <= 4096: 3-6% at M = K = 4096).
// For one or two batch rows the reuse path runs the streaming kernel above
// with NB = B instead (each decoded weight still serves every batch row):
// 16 batch columns of MFMA operands cost more activation traffic than they
// save there.
// ---------------------------------------------------------------------------
constexpr int kReuseBatch = 16;

__host__ __device__ constexpr size_t reuse_lds_bytes_for(int ks, int K, bool staged) {
  return (size_t)ks * 256 * sizeof(float) +
         (staged ? (size_t)16 * (K / kGroupSize) * sizeof(uint16_t) : 0);
}

template <int KS, int UG, bool kStaged>
__global__ __launch_bounds__(KS * 64) void gemv_reuse(const uint4* __restrict__ packed,
                                                      const uint16_t* __restrict__ scales,
                                                      const uint4* __restrict__ x4,
                                                      uint16_t* __restrict__ y, int M, int K,
                                                      int B) {
  static_assert(!kStaged || UG == 1, "the staged variant takes one group per iteration");
  write_stamp(DK_STAMP_REUSE);
  extern __shared__ float lds_reuse[];
  const int G = K >> 7;
  const int nck = K >> 5;
  float* red = lds_reuse;                                             // [KS][64][4]
  uint16_t* sT = reinterpret_cast<uint16_t*>(lds_reuse + KS * 256);   // [G][16], staged only

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row0 = blockIdx.x * 16;
  const int b0 = blockIdx.y * kReuseBatch;

  if (kStaged) {
    // sT[g][r] = scales[row0 + r][g].
    for (int e = threadIdx.x; e < 16 * G; e += blockDim.x) {
      const int r = e / G, g = e - r * G;
      const int row = min(row0 + r, M - 1);
      sT[g * 16 + r] = scales[(size_t)row * G + g];
    }
    __syncthreads();
  }

  const int r_lane = lane & 15;  // A row / B batch column
  const int kq = lane >> 4;      // lane group: 16-byte quarter of a group
  const int b = b0 + r_lane;
  const int rows = min(16, M - row0);
  const auto rw = buffer_rsrc(packed + (size_t)row0 * nck, (uint32_t)(rows * (K / 2)));
  const auto rs = buffer_rsrc(scales + (size_t)row0 * G, (uint32_t)(rows * G * 2));
  const auto rx = buffer_rsrc(x4, (uint32_t)((size_t)B * K * 2));
  const int xbase = b < B ? b * K * 2 + kq * 64 : kOutOfRange;
  const int wbase = (r_lane * nck + kq) * 16;

  f4_t acc = {0.f, 0.f, 0.f, 0.f};
  for (int g0 = wave; g0 < G; g0 += KS * UG) {
    uint4 xv[UG][4];
    uint4 w[UG];
    float sc[UG][4];
#pragma unroll
    for (int u = 0; u < UG; ++u) {
      const int g = g0 + u * KS;
      const int xo = (b < B && g < G) ? xbase + g * 256 : kOutOfRange;
#pragma unroll
      for (int j = 0; j < 4; ++j) xv[u][j] = buffer_load16<0>(rx, xo + 16 * j);
    }
    if (!kStaged) {
#pragma unroll
      for (int u = 0; u < UG; ++u) {
        const int g = g0 + u * KS;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int off = g < G ? ((4 * kq + v) * G + g) * 2 : kOutOfRange;
          sc[u][v] = h2f(__builtin_amdgcn_raw_buffer_load_b16(rs, off, 0, 0));
        }
      }
    }
#pragma unroll
    for (int u = 0; u < UG; ++u) {
      const int g = g0 + u * KS;
      w[u] = buffer_load16<kLoadNonTemporal>(rw, g < G ? wbase + g * 64 : kOutOfRange);
    }
    // Direct path: every load of the stage is issued before the first MFMA.
    // Left to itself the scheduler moves the second group's activation loads
    // behind the first group's MFMAs, which makes them wait for its weights
    // (4.87 vs 5.48 us for 8 waves x 2 groups at M = K = 4096, B = 2).
    if constexpr (!kStaged) __builtin_amdgcn_sched_barrier(0);
    if (kStaged) {
      const uint2 s4 = *reinterpret_cast<const uint2*>(sT + g0 * 16 + 4 * kq);
      sc[0][0] = h2f((uint16_t)(s4.x & 0xFFFFu));
      sc[0][1] = h2f((uint16_t)(s4.x >> 16));
      sc[0][2] = h2f((uint16_t)(s4.y & 0xFFFFu));
      sc[0][3] = h2f((uint16_t)(s4.y >> 16));
    }
#pragma unroll
    for (int u = 0; u < UG; ++u) {
      const uint32_t words[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
      f4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j)
        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(unpack_word_h8(words[j]), pair_x8(xv[u][j]), c,
                                                   0, 0, 0);
      // A group past G loaded zeros (weights, and scales on the direct path),
      // so it adds nothing.
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[v] = __builtin_fmaf(c[v], sc[u][v], acc[v]);
    }
  }

  // Cross-wave reduction of the 16x16 tile, in wave order.
#pragma unroll
  for (int v = 0; v < 4; ++v) red[(wave * 64 + lane) * 4 + v] = acc[v];
  __syncthreads();
  if (wave == 0) {
    f4_t t = {0.f, 0.f, 0.f, 0.f};
    for (int w2 = 0; w2 < KS; ++w2)
#pragma unroll
      for (int v = 0; v < 4; ++v) t[v] += red[(w2 * 64 + lane) * 4 + v];
    if (b < B) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int orow = row0 + 4 * kq + v;
        if (orow < M) y[(size_t)b * M + orow] = f2h(t[v]);
      }
    }
  }
}

}  // namespace dk
