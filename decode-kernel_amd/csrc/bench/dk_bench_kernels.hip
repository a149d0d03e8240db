// Measurement-only kernels for the benchmark tools (dk_bench), built into
// dk_bench/libdk_bench.so and never linked into the product library.
//
//  * read-floor probes: one pass over a buffer with L 16-byte loads per lane
//    all issued before the first wait, over a chosen grid, with or without
//    the non-temporal hint: the fastest a kernel that only reads N bytes can
//    run on this part, per launch;
//  * the load-only ablation of the streaming GEMV: the product kernel
//    (gemv_v5_lds) with its decode and products replaced (same loads, LDS
//    stages, grid and reduction), to separate the arithmetic from the
//    bandwidth (the open question of the reference's README.md:44);
//  * one-stage GEMV variants for short rows (K <= 4096): activations through
//    LDS or per wave in registers, weights issued first or last, one or two
//    waves per row;
//  * split-K over workgroups with a ticket reduction (gemv_v4_lds, the form
//    the product's v4 replaced), including an instance that stores its
//    partials and stops, which prices the cross-workgroup reduction, and the
//    product's split-over-waves v4 at every shape the v4 sweep times;
//  * timestamps on the GPU's wall clock for the benchmark timer.
// Outputs of the ablation kernels are meaningless by design; every other
// kernel here computes the GEMV (checked against the product by the tools).
#include <hip/hip_runtime.h>

#include <atomic>

#include "dk_kernels.hpp"
#include "dk_mlp.hpp"

#define DKB_API extern "C" __attribute__((visibility("default")))

namespace dkb {

using namespace dk;

// ---------------------------------------------------------------------------
// Read-floor probe. Lane g of the grid (g = block * T + thread) reads 16-byte
// pieces g, g + P, ..., g + (L - 1) P of each pass, P = G T lanes, all L
// loads issued before the first is used; passes repeat until the buffer
// ends. Pieces past the end read zero (out-of-range buffer offsets). Each
// wave writes one fp32 sum to partials[block * T / 64 + wave].
// ---------------------------------------------------------------------------
template <int L, bool kNt>
__global__ __launch_bounds__(1024) void read_probe(const uint4* __restrict__ src, unsigned bytes,
                                                   float* __restrict__ partials) {
  const auto r = buffer_rsrc(src, bytes);
  const unsigned P = gridDim.x * blockDim.x;
  const unsigned g = blockIdx.x * blockDim.x + threadIdx.x;
  const unsigned pieces = bytes / 16;
  float a = 0.f;
  for (unsigned base = 0; base < pieces; base += P * L) {
    uint4 v[L];
#pragma unroll
    for (int i = 0; i < L; ++i) {
      const unsigned p = base + g + (unsigned)i * P;
      v[i] = buffer_load16<kNt ? kLoadNonTemporal : 0>(r, p < pieces ? (int)(p * 16) : kOutOfRange);
    }
#pragma unroll
    for (int i = 0; i < L; ++i)
      a += __builtin_bit_cast(float, v[i].x ^ v[i].y) + __builtin_bit_cast(float, v[i].z ^ v[i].w);
  }
  a = wave_sum(a);
  if ((threadIdx.x & 63) == 63) partials[(blockIdx.x * blockDim.x + threadIdx.x) / 64] = a;
}

// ---------------------------------------------------------------------------
// Ablation maths for the stage loop (see StageMath). Both keep every load of
// the product kernel live by folding the loaded words into the result.
//  NoDecode: reads the stage's activation pieces from LDS as the product
//            does and XOR-folds them with the weight words (two logic ops
//            per word instead of the decode and four v_dot2);
//  LoadsOnly: folds only the weight words and scales (no LDS reads).
// ---------------------------------------------------------------------------
struct MathNoDecode {
  template <int R, int U, int W, int NB, typename Layout, int kS>
  static __device__ __forceinline__ void compute(const LdsStage<R, U, W, NB, kS>& st,
                                                 const uint4 (&xs)[LdsActsT<kS * U, NB>::kSlots],
                                                 float (&acc)[NB][R], int lane, int sl) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        uint32_t h[R];
#pragma unroll
        for (int r = 0; r < R; ++r) h[r] = 0u;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint4 pv = xs[((b * kS * U + sl * U + u) * 4 + j) * kWave + lane];
          const uint32_t xw = pv.x ^ pv.y ^ pv.z ^ pv.w;
#pragma unroll
          for (int r = 0; r < R; ++r) {
            const uint32_t words[4] = {st.w[u][r].x, st.w[u][r].y, st.w[u][r].z, st.w[u][r].w};
            h[r] ^= words[j] ^ xw;
          }
        }
#pragma unroll
        for (int r = 0; r < R; ++r)
          acc[b][r] += h2f((uint16_t)st.s[u][r]) * (float)(h[r] & 0xFFu);
      }
  }
};

struct MathLoadsOnly {
  template <int R, int U, int W, int NB, typename Layout, int kS>
  static __device__ __forceinline__ void compute(const LdsStage<R, U, W, NB, kS>& st,
                                                 const uint4 (&)[LdsActsT<kS * U, NB>::kSlots],
                                                 float (&acc)[NB][R], int, int) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const uint32_t h = st.w[u][r].x ^ st.w[u][r].y ^ st.w[u][r].z ^ st.w[u][r].w;
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[b][r] += h2f((uint16_t)st.s[u][r]) * (float)(h & 0xFFu);
      }
  }
};

// ---------------------------------------------------------------------------
// One-stage GEMV for rows of up to S * U * 2048 weights, one batch row: each
// row is taken by S waves (wave s of the row takes chunks [64 U s, 64 U
// (s + 1)), lane l its chunks 64 U s + 64 u + l), W waves per workgroup, so
// W / S rows per workgroup. kLds: the workgroup loads the activations once,
// pairs them and shares them through LDS (the product's stage); otherwise
// each wave loads its own chunks' activations (four 16-byte loads per chunk,
// L1/L2 hits after the first wave) and pairs them in registers.
// kWeightsFirst: the weight loads issue before the activation and scale
// loads (with LDS the publish then waits for the weights too: loads return
// in order). With S = 2 the two halves' fp32 sums are added in wave order
// through LDS. Workgroups are renumbered per XCD as in v5.
// ---------------------------------------------------------------------------
template <int U, int W, int S, bool kLds, bool kWeightsFirst>
__global__ __launch_bounds__(W * kWave) void gemv_onestage(const uint4* __restrict__ packed,
                                                           const uint16_t* __restrict__ scales,
                                                           const uint4* __restrict__ x4,
                                                           uint16_t* __restrict__ y, int M, int K) {
  static_assert(W % S == 0, "whole rows per workgroup");
  constexpr int kRowsPerWg = W / S;
  constexpr int kChunks = S * U * kWave;  // chunks of one stage (the whole row)
  __shared__ uint4 xs[kLds ? kChunks * 4 : 1];
  __shared__ float red[W];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wg = xcd_contiguous_block(blockIdx.x, (M + kRowsPerWg - 1) / kRowsPerWg);
  const int row = wg * kRowsPerWg + wave % kRowsPerWg;
  const int half = wave / kRowsPerWg;  // which part of the row this wave takes
  const bool active = row < M;
  const int nck = K >> 5;
  const int G = K >> 7;
  const auto rw = buffer_rsrc(packed + (size_t)(active ? row : 0) * nck, active ? (uint32_t)(K / 2) : 0u);
  const auto rs = buffer_rsrc(scales + (size_t)(active ? row : 0) * G, active ? (uint32_t)(G * 2) : 0u);
  const auto rx = buffer_rsrc(x4, (uint32_t)(K * 2));

  uint4 w[U];
  uint32_t sc[U];
  uint4 xv[kLds ? (kChunks * 4 + W * kWave - 1) / (W * kWave) : 4 * U];
  constexpr int kXLoads = sizeof(xv) / sizeof(uint4);
  auto load_w = [&]() {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = (half * U + u) * kWave + lane;
      sc[u] = __builtin_amdgcn_raw_buffer_load_b16(rs, c < nck ? (c >> 2) * 2 : kOutOfRange, 0, 0);
      w[u] = buffer_load16<kLoadNonTemporal>(rw, c < nck ? c * 16 : kOutOfRange);
    }
  };
  auto load_x = [&]() {
#pragma unroll
    for (int i = 0; i < kXLoads; ++i) {
      if constexpr (kLds) {
        const int piece = tid + i * W * kWave;  // 16-byte piece of the row's activations
        xv[i] = buffer_load16<0>(rx, piece < kChunks * 4 && (piece >> 2) < nck ? piece * 16 : kOutOfRange);
      } else {
        const int c = (half * U + i / 4) * kWave + lane;
        xv[i] = buffer_load16<0>(rx, c < nck ? (c * 4 + (i & 3)) * 16 : kOutOfRange);
      }
    }
  };
  if constexpr (kWeightsFirst) {
    load_w();
    load_x();
  } else {
    load_x();
    load_w();
  }
  __builtin_amdgcn_sched_barrier(0);
  h2_t xp[U][4][4];
  if constexpr (kLds) {
#pragma unroll
    for (int i = 0; i < kXLoads; ++i) {
      const int piece = tid + i * W * kWave;
      if (piece < kChunks * 4) {
        h2_t p[4];
        pair_x(xv[i], p);
        // slot (chunk c, piece j) at (j * kChunks + c): lane-consecutive reads
        xs[(piece & 3) * kChunks + (piece >> 2)] =
            make_uint4(__builtin_bit_cast(uint32_t, p[0]), __builtin_bit_cast(uint32_t, p[1]),
                       __builtin_bit_cast(uint32_t, p[2]), __builtin_bit_cast(uint32_t, p[3]));
      }
    }
    lds_barrier();
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint4 pv = xs[j * kChunks + (half * U + u) * kWave + lane];
        xp[u][j][0] = as_h2(pv.x);
        xp[u][j][1] = as_h2(pv.y);
        xp[u][j][2] = as_h2(pv.z);
        xp[u][j][3] = as_h2(pv.w);
      }
  } else {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j) pair_x(xv[4 * u + j], xp[u][j]);
  }
  float acc = 0.f;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t words[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
    float part = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) part = dot_word(words[j], xp[u][j], part);
    acc = __builtin_fmaf(part, h2f((uint16_t)sc[u]), acc);
  }
  const float t = wave_sum(acc);
  if constexpr (S == 1) {
    if (active && lane == 63) y[row] = f2h(t);
  } else {
    if (lane == 63) red[wave] = t;
    __syncthreads();
    if (half == 0 && active && lane == 63) {
      float sum = 0.f;
#pragma unroll
      for (int s = 0; s < S; ++s) sum += red[s * kRowsPerWg + wave];
      y[row] = f2h(sum);
    }
  }
}

// ---------------------------------------------------------------------------
// Split-K over workgroups, the form the product's v4 replaced (measured by
// dk_bench.levers v4 beside it). grid = (row blocks of W R rows, batch tiles
// of NB rows, S slices); workgroup (x, y, z) streams its rows over group
// slice z with the stage loop of v5 (LDS-shared activations, buffer loads
// through descriptors scoped to the slice). Each wave stores its fp32 row
// sums to partials[z][b][row] with agent-scope stores (past the non-coherent
// per-XCD L2s) and waits for them; thread 0 then takes the ticket of its
// (row block, batch tile) (take_ticket). The last of the S workgroups adds
// the S partials in slice order and writes y. kReduce 0: that reduction;
// kReduce 2: store the partials and stop, without y (prices the reduction,
// about 2 us on MI355X: the stores, the ticket and the reads each cross the
// XCDs through memory).
// ---------------------------------------------------------------------------
constexpr int kV4Tickets = 0;

template <int R, int U, int W, int NB, bool kPrefetch, int kReduce>
__global__ __launch_bounds__(W * kWave) void gemv_v4_lds(const uint4* __restrict__ packed,
                                                         const uint16_t* __restrict__ scales,
                                                         const uint4* __restrict__ x4,
                                                         uint16_t* __restrict__ y,
                                                         float* __restrict__ ws,
                                                         unsigned long long* __restrict__ tickets,
                                                         unsigned long long gen, int M, int K,
                                                         int B) {
  write_stamp(4);
  __shared__ LdsActs<U, NB> xs;
  __shared__ int last;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nblk = (M + W * R - 1) / (W * R);
  const int wg = xcd_contiguous_block(blockIdx.x, nblk);
  const int row0 = (wg * W + wave) * R;
  const bool active = row0 < M;  // wave-uniform
  const int b0 = blockIdx.y * NB;
  const int S = gridDim.z;
  const int z = blockIdx.z;
  const int nck = K >> 5;
  const int G = K >> 7;
  const int gps = (G + S - 1) / S;
  const int gbeg = min(z * gps, G);
  const int Gs = min(gbeg + gps, G) - gbeg;  // groups of this slice (0 if none)
  const int rows = active ? min(R, M - row0) : 0;
  const int rbase = active ? row0 : 0;
  // The slice of row r is chunks [4 gbeg, 4 (gbeg + Gs)) at r * nck chunks
  // from the descriptor base; the range ends after the last row's slice.
  const auto rw = buffer_rsrc(packed + (size_t)rbase * nck + (size_t)gbeg * 4,
                              rows > 0 ? (uint32_t)((rows - 1) * (K / 2) + Gs * 64) : 0u);
  const auto rs = buffer_rsrc(scales + (size_t)rbase * G + gbeg,
                              rows > 0 ? (uint32_t)(((rows - 1) * G + Gs) * 2) : 0u);
  const auto rx = buffer_rsrc(x4 + (size_t)gbeg * 16, (uint32_t)((size_t)B * K * 2 - (size_t)gbeg * 256));

  float acc[NB][R];
  lds_stream<R, U, W, NB, kPrefetch, LayoutLogical, R>(xs, acc, rw, rs, rw, rs, rx, 4 * Gs, nck, G,
                                                        K, b0, B, tid, lane);
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float t = wave_sum(acc[b][r]);
      if (active && lane == 63 && row0 + r < M && b0 + b < B) {
        const size_t o = (size_t)(b0 + b) * M + row0 + r;
        __hip_atomic_store(&ws[(size_t)z * B * M + o], t, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  if constexpr (kReduce == kV4Tickets) {
    // Every wave's partial stores are complete before the ticket is taken.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    unsigned long long* ticket = &tickets[(size_t)blockIdx.y * nblk + wg];
    if (tid == 0) last = take_ticket(ticket, gen, S);
    __syncthreads();
    if (!last) return;
    constexpr int kOut = W * R * NB;
    for (int t = tid; t < kOut; t += W * kWave) {
      const int row = wg * W * R + t % (W * R);
      const int b = b0 + t / (W * R);
      if (row >= M || b >= B) continue;
      float sum = 0.f;
      for (int s = 0; s < S; ++s)
        sum += __hip_atomic_load(&ws[((size_t)s * B + b) * M + row], __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
      y[(size_t)b * M + row] = f2h(sum);
    }
    if (tid == 0) release_ticket(ticket, gen);
  }
}

// ---------------------------------------------------------------------------
// Timestamp: one lane writes the GPU's constant-rate wall clock
// (s_memrealtime, hipDeviceAttributeWallClockRate kHz) to dst[slot] with a
// vector store. Two of them inside a captured graph bracket the launches
// between them on the GPU's own clock.
// ---------------------------------------------------------------------------
__global__ void timestamp_kernel(unsigned long long* __restrict__ dst, int slot) {
  if (threadIdx.x == 0) dst[slot] = __builtin_amdgcn_s_memrealtime();
}

}  // namespace dkb

namespace {

int launch_error(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
    return 2;
  }
  return 0;
}

}  // namespace

// Read-floor probe: `blocks` workgroups of `threads` (64..1024, multiple of
// 64) lanes, `loads` (1, 2, 4, 8) loads per lane per pass, nt = non-temporal
// hint. `partials` holds blocks * threads / 64 floats. Returns 0 or an error.
DKB_API int dkb_read_probe(const void* src, size_t bytes, float* partials, int blocks, int threads,
                           int loads, int nt, hipStream_t stream) {
  if (!src || !partials || bytes % 16 || bytes > 0x7fffffffu || blocks < 1 || threads < 64 ||
      threads > 1024 || threads % 64)
    return 1;
  const auto* s = static_cast<const uint4*>(src);
  const unsigned b = (unsigned)bytes;
#define DKB_READ(L)                                                                         \
  if (nt)                                                                                    \
    hipLaunchKernelGGL((dkb::read_probe<L, true>), dim3(blocks), dim3(threads), 0, stream, s, b, \
                       partials);                                                            \
  else                                                                                       \
    hipLaunchKernelGGL((dkb::read_probe<L, false>), dim3(blocks), dim3(threads), 0, stream, s, b, \
                       partials);
  switch (loads) {
    case 1: DKB_READ(1) break;
    case 2: DKB_READ(2) break;
    case 4: DKB_READ(4) break;
    case 8: DKB_READ(8) break;
    default: return 1;
  }
#undef DKB_READ
  return launch_error("read probe");
}

namespace {

// The streaming-kernel shapes the product uses at one batch row
// (launch_lds in dk_gemv.hip), by (R, U, W, prefetch), with the ablation
// maths. math: 0 product, 1 no decode, 2 loads only.
template <int R, int U, int W, bool PF>
int v5_math(int math, const uint4* p, const uint16_t* s, const uint4* x, uint16_t* y, int M, int K,
            hipStream_t stream) {
  const dim3 grid((M + W * R - 1) / (W * R)), block(W * 64);
  switch (math) {
    case 0:
      hipLaunchKernelGGL((dk::gemv_v5_lds<R, U, W, 1, PF, dk::LayoutLogical, 5, dk::StageMath>), grid,
                         block, 0, stream, p, s, x, y, M, K, 1);
      break;
    case 1:
      hipLaunchKernelGGL((dk::gemv_v5_lds<R, U, W, 1, PF, dk::LayoutLogical, 5, dkb::MathNoDecode>),
                         grid, block, 0, stream, p, s, x, y, M, K, 1);
      break;
    case 2:
      hipLaunchKernelGGL((dk::gemv_v5_lds<R, U, W, 1, PF, dk::LayoutLogical, 5, dkb::MathLoadsOnly>),
                         grid, block, 0, stream, p, s, x, y, M, K, 1);
      break;
    default:
      return 1;
  }
  return launch_error("v5 math");
}

}  // namespace

// The streaming GEMV at one batch row with shape (R, U, W, prefetch) and
// math 0 (product), 1 (no decode) or 2 (loads only). Returns 3 for a shape
// that is not instantiated here.
DKB_API int dkb_v5(int math, int R, int U, int W, int prefetch, const void* packed,
                   const void* scales, const void* x, void* y, int M, int K, hipStream_t stream) {
  const auto* p = static_cast<const uint4*>(packed);
  const auto* s = static_cast<const uint16_t*>(scales);
  const auto* xx = static_cast<const uint4*>(x);
  auto* yy = static_cast<uint16_t*>(y);
#define DKB_V5(r, u, w, pf)                                   \
  if (R == r && U == u && W == w && (prefetch != 0) == pf) \
    return v5_math<r, u, w, pf>(math, p, s, xx, yy, M, K, stream);
  DKB_V5(1, 1, 16, true)
  DKB_V5(1, 2, 4, true)
  DKB_V5(1, 4, 4, true)
  DKB_V5(1, 6, 4, true)
  DKB_V5(1, 4, 8, true)
  DKB_V5(2, 1, 8, true)
  DKB_V5(2, 2, 4, false)
  DKB_V5(2, 1, 8, false)
  DKB_V5(1, 2, 16, true)
  DKB_V5(2, 1, 16, true)
  DKB_V5(1, 2, 8, true)
  DKB_V5(1, 2, 8, false)
  DKB_V5(1, 2, 16, false)
  DKB_V5(1, 1, 8, true)
#undef DKB_V5
  return 3;
}

// One-stage GEMV (B = 1, K <= S * U * 2048): variant bits lds, weights_first;
// S = 1 (U = 2) or 2 (U = 1); W in {4, 8, 16}. Returns 3 if not instantiated.
DKB_API int dkb_onestage(int W, int S, int lds, int weights_first, const void* packed,
                         const void* scales, const void* x, void* y, int M, int K,
                         hipStream_t stream) {
  if (K > S * (S == 1 ? 2 : 1) * 2048 || K % 128) return 1;
  const auto* p = static_cast<const uint4*>(packed);
  const auto* s = static_cast<const uint16_t*>(scales);
  const auto* xx = static_cast<const uint4*>(x);
  auto* yy = static_cast<uint16_t*>(y);
#define DKB_ONE(w, ss, l, wf)                                                                     \
  if (W == w && S == ss && (lds != 0) == l && (weights_first != 0) == wf) {                       \
    hipLaunchKernelGGL((dkb::gemv_onestage<ss == 1 ? 2 : 1, w, ss, l, wf>),                      \
                       dim3((M + w / ss - 1) / (w / ss)), dim3(w * 64), 0, stream, p, s, xx, yy, M, K); \
    return launch_error("onestage");                                                              \
  }
#define DKB_ONE4(w, ss) DKB_ONE(w, ss, true, false) DKB_ONE(w, ss, true, true) \
                        DKB_ONE(w, ss, false, false) DKB_ONE(w, ss, false, true)
  DKB_ONE4(4, 1)
  DKB_ONE4(8, 1)
  DKB_ONE4(16, 1)
  DKB_ONE4(8, 2)
  DKB_ONE4(16, 2)
#undef DKB_ONE4
#undef DKB_ONE
  return 3;
}

// Split-K instances for the v4 shape sweep (B = 1): shape (R, U, W,
// prefetch), S slices, reduce 0 (tickets: the product's), 2 (partials only:
// no ticket and no y; prices the reduction). `tickets` holds ceil(M / (W R))
// 8-byte tickets, `ws` [S, M] floats; gen as for the product (low 6 bits 0).
DKB_API int dkb_v4(int R, int U, int W, int prefetch, int reduce, int S, const void* packed,
                   const void* scales, const void* x, void* y, float* ws, void* tickets,
                   unsigned long long gen, int M, int K, hipStream_t stream) {
  const auto* p = static_cast<const uint4*>(packed);
  const auto* s = static_cast<const uint16_t*>(scales);
  const auto* xx = static_cast<const uint4*>(x);
  auto* yy = static_cast<uint16_t*>(y);
  auto* t = static_cast<unsigned long long*>(tickets);
  if (S < 1 || S > 32) return 1;
#define DKB_V4(r, u, w, pf, red)                                                                  \
  if (R == r && U == u && W == w && (prefetch != 0) == pf && reduce == red) {                    \
    hipLaunchKernelGGL((dkb::gemv_v4_lds<r, u, w, 1, pf, red>), dim3((M + w * r - 1) / (w * r), 1, S), \
                       dim3(w * 64), 0, stream, p, s, xx, yy, ws, t, gen, M, K, 1);              \
    return launch_error("v4");                                                                    \
  }
#define DKB_V4R(r, u, w, pf) DKB_V4(r, u, w, pf, 0) DKB_V4(r, u, w, pf, 2)
  DKB_V4R(1, 1, 4, true)
  DKB_V4R(1, 2, 4, true)
  DKB_V4R(1, 4, 4, true)
  DKB_V4R(1, 1, 8, true)
  DKB_V4R(1, 2, 8, true)
  DKB_V4R(1, 4, 8, true)
  DKB_V4R(1, 2, 4, false)
  DKB_V4R(1, 4, 4, false)
  DKB_V4R(2, 1, 4, true)
  DKB_V4R(2, 2, 4, true)
  DKB_V4R(1, 1, 16, true)
  DKB_V4R(1, 2, 16, true)
#undef DKB_V4R
#undef DKB_V4
  return 3;
}

// Writes the wall clock to ((uint64_t*)dst)[slot] on `stream`.
DKB_API int dkb_timestamp(void* dst, int slot, hipStream_t stream) {
  if (!dst || slot < 0) return 1;
  hipLaunchKernelGGL(dkb::timestamp_kernel, dim3(1), dim3(64), 0, stream,
                     static_cast<unsigned long long*>(dst), slot);
  return launch_error("timestamp");
}

// Rate of the clock dkb_timestamp reads, in kHz, for the current device
// (<= 0 on error).
DKB_API int dkb_wall_clock_khz(void) {
  int dev = 0, khz = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess) return -1;
  return khz;
}

// The reuse path's tile kernels at any instantiated shape (B rows in tiles of
// 16): kind 0 gemv_reuse<KS, RT, SG, pairs> (MFMA operands loaded directly),
// kind 1 gemv_reuse_lds<KS, RT, pairs, SG> (both operands staged in LDS by
// the buffer-load-to-LDS path, blocks of SG = 2 or 4 groups). Returns 3 (nothing launched) for a
// shape not instantiated here.
DKB_API int dkb_reuse(int kind, int KS, int RT, int SG, int pairs, const void* packed,
                      const void* scales, const void* x, void* y, int M, int K, int B,
                      hipStream_t stream) {
  const auto* p = static_cast<const uint4*>(packed);
  const auto* s = static_cast<const uint16_t*>(scales);
  const auto* xx = static_cast<const uint4*>(x);
  auto* yy = static_cast<uint16_t*>(y);
#define DKB_R0(ks, rt, sg, pr)                                                                 \
  if (kind == 0 && KS == ks && RT == rt && SG == sg && pairs == (int)pr) {                     \
    hipLaunchKernelGGL((dk::gemv_reuse<ks, rt, sg, pr>), dim3((M + 16 * rt - 1) / (16 * rt),     \
                       (B + 15) / 16), dim3(ks * 64), 0, stream, p, s, xx, yy, M, K, B);        \
    return launch_error("reuse");                                                              \
  }
#define DKB_R1S(ks, rt, pr, sg)                                                                \
  if (kind == 1 && KS == ks && RT == rt && SG == sg && pairs == (int)pr) {                     \
    hipLaunchKernelGGL((dk::gemv_reuse_lds<ks, rt, pr, sg>), dim3((M + 16 * rt - 1) / (16 * rt), \
                       (B + 15) / 16), dim3(ks * 64), 0, stream, p, s, xx, yy, M, K, B);        \
    return launch_error("reuse lds");                                                          \
  }
#define DKB_R1(ks, rt, pr) DKB_R1S(ks, rt, pr, 2)
#define DKB_R2(ks, rt)                                                                         \
  if (kind == 2 && KS == ks && RT == rt && SG == 2 && pairs) {                                 \
    hipLaunchKernelGGL((dk::gemv_reuse_pf<ks, rt>), dim3((M + 16 * rt - 1) / (16 * rt),        \
                       (B + 15) / 16), dim3(ks * 64), 0, stream, p, s, xx, yy, M, K, B);        \
    return launch_error("reuse pf");                                                           \
  }
  DKB_R2(4, 1) DKB_R2(6, 1) DKB_R2(7, 1) DKB_R2(4, 2) DKB_R2(6, 2)
#undef DKB_R2
#define DKB_RX(kd, ks, rt, xl)                                                                 \
  if (kind == kd && KS == ks && RT == rt && SG == 2 && pairs && B <= 2 * xl) {                 \
    hipLaunchKernelGGL((dk::gemv_reuse_pf<ks, rt, xl>), dim3((M + 16 * rt - 1) / (16 * rt), 1), \
                       dim3(ks * 64), 0, stream, p, s, xx, yy, M, K, B);                       \
    return launch_error("reuse pf");                                                           \
  }
  DKB_RX(3, 4, 1, 4) DKB_RX(3, 6, 1, 4) DKB_RX(4, 4, 1, 2) DKB_RX(4, 6, 1, 2) DKB_RX(3, 4, 2, 4)
  DKB_RX(3, 6, 2, 4) DKB_RX(3, 8, 1, 4) DKB_RX(3, 8, 2, 4)
#undef DKB_RX
  DKB_R0(8, 1, 2, true) DKB_R0(8, 1, 2, false) DKB_R0(8, 1, 4, false) DKB_R0(16, 1, 4, false)
  DKB_R0(16, 1, 2, false) DKB_R0(8, 2, 2, true) DKB_R0(8, 2, 2, false) DKB_R0(8, 2, 4, false)
  DKB_R1(8, 1, true) DKB_R1(8, 1, false) DKB_R1(16, 1, true) DKB_R1(16, 1, false)
  DKB_R1(8, 2, true) DKB_R1(8, 2, false) DKB_R1(4, 1, true) DKB_R1(4, 2, true)
  DKB_R1S(8, 1, true, 4) DKB_R1S(4, 1, true, 4) DKB_R1S(4, 2, true, 4) DKB_R1S(8, 1, false, 4)
#undef DKB_R1
#undef DKB_R1S
#undef DKB_R0
  return 3;
}

// The split-K tile kernels (B rows in tiles of 16, S slices of each row):
// kind 0 gemv_reuse_split<KS, RT, 2> (MFMA operands loaded directly), kind 1
// gemv_reuse_split_pf<KS, RT> (double-buffered LDS staging; an even number
// of groups per row and 4-byte aligned scales). workspace: one 8-byte
// ticket per set of RT tiles and batch tile, padded to 256 bytes, then
// S * B * M fp32 partials. Returns 3 (nothing launched) for a shape not
// instantiated here.
DKB_API size_t dkb_reuse_split_workspace(int RT, int S, int M, int B) {
  const size_t tickets = (size_t)((M + 16 * RT - 1) / (16 * RT)) * (size_t)((B + 15) / 16);
  return (tickets * 8 + 255) / 256 * 256 + (size_t)S * B * M * sizeof(float);
}

DKB_API int dkb_reuse_split(int kind, int KS, int RT, int S, const void* packed, const void* scales,
                            const void* x, void* y, void* workspace, int M, int K, int B,
                            hipStream_t stream) {
  static std::atomic<unsigned long long> gens{0x5bd1e9955bd1e995ull};
  const auto* p = static_cast<const uint4*>(packed);
  const auto* s = static_cast<const uint16_t*>(scales);
  const auto* xx = static_cast<const uint4*>(x);
  auto* yy = static_cast<uint16_t*>(y);
  const size_t tickets = (size_t)((M + 16 * RT - 1) / (16 * RT)) * (size_t)((B + 15) / 16);
  auto* tk = static_cast<unsigned long long*>(workspace);
  auto* part = reinterpret_cast<float*>(static_cast<char*>(workspace) + (tickets * 8 + 255) / 256 * 256);
  const unsigned long long gen =
      (gens.fetch_add(1ull, std::memory_order_relaxed) & ((1ull << 58) - 1ull)) << 6;
  const dim3 grid((M + 16 * RT - 1) / (16 * RT), (B + 15) / 16, S);
  if (S < 1 || S > 63) return 2;
#define DKB_S(kd, ks, rt, kernel)                                                              \
  if (kind == kd && KS == ks && RT == rt) {                                                    \
    hipLaunchKernelGGL((kernel), grid, dim3(ks * 64), 0, stream, p, s, xx, yy, part, tk, gen, M, \
                       K, B);                                                                  \
    return launch_error("reuse split");                                                        \
  }
  DKB_S(0, 8, 2, (dk::gemv_reuse_split<8, 2, 2>))
  DKB_S(1, 4, 1, (dk::gemv_reuse_split_pf<4, 1>))
  DKB_S(1, 6, 1, (dk::gemv_reuse_split_pf<6, 1>))
  DKB_S(1, 4, 2, (dk::gemv_reuse_split_pf<4, 2>))
#undef DKB_S
  return 3;
}

// The fused gate/up tile kernels at any instantiated shape (B rows in tiles
// of 16): kind 0 gate_up_silu_tiles<KS, 2, pairs> (MFMA operands loaded
// directly), kind 1 gate_up_silu_tiles_lds<KS, pairs> (both operands staged
// in LDS), kind 2 gate_up_silu_tiles_pf<KS> (staged and double buffered;
// pairs only), kind 3 gate_up_silu_tiles_pf<KS, 4> (4 x loads per block, up
// to 8 batch rows). Returns 3 (nothing launched) for a shape not
// instantiated here.
DKB_API int dkb_gate_up(int kind, int KS, int pairs, const void* gate, const void* gate_scales,
                        const void* up, const void* up_scales, const void* x, void* h, int I, int H,
                        int B, hipStream_t stream) {
  const auto* g = static_cast<const uint4*>(gate);
  const auto* gs = static_cast<const uint16_t*>(gate_scales);
  const auto* u = static_cast<const uint4*>(up);
  const auto* us = static_cast<const uint16_t*>(up_scales);
  const auto* xx = static_cast<const uint4*>(x);
  auto* hh = static_cast<uint16_t*>(h);
  const dim3 grid((I + 15) / 16, (B + 15) / 16);
#define DKB_GU(kd, ks, pr, kernel)                                                              \
  if (kind == kd && KS == ks && pairs == (int)pr) {                                            \
    hipLaunchKernelGGL(kernel, grid, dim3(ks * 64), 0, stream, g, gs, u, us, xx, I, H, B, hh); \
    return launch_error("gate/up tiles");                                                      \
  }
  DKB_GU(0, 8, true, (dk::gate_up_silu_tiles<8, 2, true>))
  DKB_GU(0, 8, false, (dk::gate_up_silu_tiles<8, 2, false>))
  DKB_GU(1, 8, true, (dk::gate_up_silu_tiles_lds<8, true>))
  DKB_GU(1, 4, true, (dk::gate_up_silu_tiles_lds<4, true>))
  DKB_GU(2, 4, true, (dk::gate_up_silu_tiles_pf<4>))
  DKB_GU(2, 6, true, (dk::gate_up_silu_tiles_pf<6>))
  if (B <= 8) {
    DKB_GU(3, 4, true, (dk::gate_up_silu_tiles_pf<4, 4>))
    DKB_GU(3, 6, true, (dk::gate_up_silu_tiles_pf<6, 4>))
  }
#undef DKB_GU
  return 3;
}

// The product's split-K kernel (gemv_v4_split, B = 1) at shape R rows per
// wave, U chunks per lane per stage, W waves, S slices per row, prefetch on
// or off; math 0 is the product's, 1 no decode and 2 loads only (as for
// dkb_v5; those at the shapes the v5 dispatch takes it for). Returns 3
// (nothing launched) for a shape not instantiated here.
DKB_API int dkb_v4s(int math, int R, int U, int W, int S, int pf, const void* packed,
                    const void* scales, const void* x, void* y, int M, int K, hipStream_t stream) {
  const auto* p = static_cast<const uint4*>(packed);
  const auto* s = static_cast<const uint16_t*>(scales);
  const auto* xx = static_cast<const uint4*>(x);
  auto* yy = static_cast<uint16_t*>(y);
#define DKB_V4S_M(mi, Mt, r, u, w, k, f)                                                        \
  if (math == mi && R == r && U == u && W == w && S == k && pf == (int)f) {                     \
    const int rows = w / k * r;                                                                 \
    hipLaunchKernelGGL((dk::gemv_v4_split<r, u, w, k, 1, f, Mt>), dim3((M + rows - 1) / rows),   \
                       dim3(w * 64), 0, stream, p, s, xx, yy, static_cast<float*>(nullptr), M, K, \
                       1, 4);                                                                   \
    return launch_error("v4 split");                                                            \
  }
#define DKB_V4S_PF(r, u, w, k, f) DKB_V4S_M(0, dk::StageMath, r, u, w, k, f)
#define DKB_V4S(r, u, w, k) DKB_V4S_PF(r, u, w, k, true) DKB_V4S_PF(r, u, w, k, false)
#define DKB_V4S_W(r, u, k) DKB_V4S(r, u, 4, k) DKB_V4S(r, u, 8, k) DKB_V4S(r, u, 16, k)
  DKB_V4S_W(1, 1, 2) DKB_V4S_W(1, 2, 2) DKB_V4S_W(1, 4, 2) DKB_V4S_W(2, 1, 2) DKB_V4S_W(2, 2, 2)
  DKB_V4S_W(1, 1, 4) DKB_V4S_W(1, 2, 4) DKB_V4S_W(2, 1, 4) DKB_V4S_W(2, 2, 4)
  DKB_V4S(1, 1, 8, 8) DKB_V4S(1, 1, 16, 8) DKB_V4S(2, 1, 8, 8) DKB_V4S(2, 1, 16, 8)
#define DKB_V4S_ABL(r, u, w, k, f) \
  DKB_V4S_M(1, dkb::MathNoDecode, r, u, w, k, f) DKB_V4S_M(2, dkb::MathLoadsOnly, r, u, w, k, f)
  DKB_V4S_ABL(1, 1, 4, 2, true) DKB_V4S_ABL(1, 2, 8, 4, true) DKB_V4S_ABL(1, 2, 8, 4, false)
  DKB_V4S_ABL(2, 2, 8, 4, false) DKB_V4S_ABL(1, 1, 16, 2, true) DKB_V4S_ABL(2, 1, 16, 2, true)
  DKB_V4S_ABL(2, 2, 8, 2, false)
#undef DKB_V4S_ABL
#undef DKB_V4S_W
#undef DKB_V4S
#undef DKB_V4S_PF
#undef DKB_V4S_M
  return 3;
}
