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
//    the same for the split-K kernel (gemv_v4_split) at the shapes the v5
//    dispatch takes it for;
//  * timestamps on the GPU's wall clock for the benchmark timer, and a
//    shader-clock probe that converts SCLK-cycle counters to time.
// Outputs of the ablation kernels are meaningless by design; the product
// maths here computes the GEMV (checked against the product by the tools).
#include <hip/hip_runtime.h>

#include <cstdio>

#include "dk_kernels.hpp"

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
// Timestamp: one lane writes the GPU's constant-rate wall clock
// (s_memrealtime, hipDeviceAttributeWallClockRate kHz) to dst[slot] with a
// vector store. Two of them inside a captured graph bracket the launches
// between them on the GPU's own clock.
// ---------------------------------------------------------------------------
__global__ void timestamp_kernel(unsigned long long* __restrict__ dst, int slot) {
  if (threadIdx.x == 0) dst[slot] = __builtin_amdgcn_s_memrealtime();
}

// Shader-clock probe: every wave runs `iters` steps of a dependent integer
// chain and workgroup 0's first wave records the shader-clock counter
// (s_memtime, in SCLK cycles) and the wall clock (s_memrealtime) before and
// after it: out[0..3] = {sclk start, sclk end, wall start, wall end}, and
// out[4] keeps the chain's result live. The SCLK rate is the ratio of the
// two intervals times the wall clock's rate; counters such as SQ_BUSY_CYCLES
// are kept in SCLK cycles.
__global__ void clock_probe_kernel(unsigned long long* __restrict__ out, int iters) {
  const unsigned long long c0 = __builtin_amdgcn_s_memtime();
  const unsigned long long w0 = __builtin_amdgcn_s_memrealtime();
  unsigned v = threadIdx.x + blockIdx.x;
  for (int i = 0; i < iters; ++i) v = v * 1664525u + 1013904223u;
  const unsigned long long c1 = __builtin_amdgcn_s_memtime();
  const unsigned long long w1 = __builtin_amdgcn_s_memrealtime();
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    out[0] = c0;
    out[1] = c1;
    out[2] = w0;
    out[3] = w1;
  }
  if (blockIdx.x == 0 && threadIdx.x == 1) out[4] = v;
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

// Writes the wall clock to ((uint64_t*)dst)[slot] on `stream`.
DKB_API int dkb_timestamp(void* dst, int slot, hipStream_t stream) {
  if (!dst || slot < 0) return 1;
  hipLaunchKernelGGL(dkb::timestamp_kernel, dim3(1), dim3(64), 0, stream,
                     static_cast<unsigned long long*>(dst), slot);
  return launch_error("timestamp");
}

// Shader-clock probe (clock_probe_kernel): `blocks` workgroups of 64 lanes,
// `iters` chain steps each; out holds 5 uint64.
DKB_API int dkb_clock_probe(void* out, int iters, int blocks, hipStream_t stream) {
  if (!out || iters < 0 || blocks < 1 || blocks > 65536) return 1;
  hipLaunchKernelGGL(dkb::clock_probe_kernel, dim3(blocks), dim3(64), 0, stream,
                     static_cast<unsigned long long*>(out), iters);
  return launch_error("clock probe");
}

// Rate of the clock dkb_timestamp reads, in kHz, for the current device
// (<= 0 on error).
DKB_API int dkb_wall_clock_khz(void) {
  int dev = 0, khz = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess) return -1;
  return khz;
}

// The product's split-K kernel (gemv_v4_split, B = 1) at shape R rows per
// wave, U chunks per lane per stage, W waves, S slices per row, prefetch on
// or off, at the shapes the v5 dispatch takes it for; math 0 is the
// product's, 1 no decode and 2 loads only (as for dkb_v5). Returns 3
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
                       1);                                                                      \
    return launch_error("v4 split");                                                            \
  }
#define DKB_V4S_ABL(r, u, w, k, f)                                                         \
  DKB_V4S_M(0, dk::StageMath, r, u, w, k, f) DKB_V4S_M(1, dkb::MathNoDecode, r, u, w, k, f) \
  DKB_V4S_M(2, dkb::MathLoadsOnly, r, u, w, k, f)
  DKB_V4S_ABL(1, 1, 4, 2, true) DKB_V4S_ABL(1, 2, 8, 4, true) DKB_V4S_ABL(1, 2, 8, 4, false)
  DKB_V4S_ABL(2, 2, 8, 4, false) DKB_V4S_ABL(1, 1, 16, 2, true) DKB_V4S_ABL(2, 1, 16, 2, true)
  DKB_V4S_ABL(2, 2, 8, 2, false)
#undef DKB_V4S_ABL
#undef DKB_V4S_M
  return 3;
}
