// W4A16 decode GEMV for MI355X (gfx950, CDNA4, wave64).
//
// One translation unit holds every GEMV variant, the dispatch stamps and the
// C ABI declared in include/decode_kernel/dk_gemv.h. The variants keep the
// reference's numbering and stamps (csrc/gemv_w4a16.cu:67-413) but each is
// written for CDNA4: wave64 lanes, 16-byte coalesced loads, whole-word nibble
// decode with packed fp16 math, v_dot2_f32_f16 or MFMA products with fp32
// accumulation, DPP wave reductions and a single-launch split-K.
//
// The kernels themselves are in dk_kernels.hpp; the fused gate/up kernel of
// the MLP decode step (dk_mlp.h) is in dk_mlp.hpp and shares the stamps.
#include <hip/hip_runtime.h>

#include <cxxabi.h>
#include <dlfcn.h>

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <string>
#include <type_traits>

#include "dk_host.hpp"
#include "dk_kernels.hpp"
#include "dk_mlp.hpp"
#include "decode_kernel/dk_gemv.h"
#include "decode_kernel/dk_mlp.h"

// ===========================================================================
// Host side: validation, launch selection and the C ABI.
// ===========================================================================
namespace dk {

thread_local std::string g_err;

int set_error(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_error(hipError_t e, const char* what) {
  return set_error(DK_ERR_HIP, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_error(e, what);
  return DK_OK;
}

}  // namespace dk

namespace {

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  return dk::set_error(code, "%s", buf);
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

constexpr int kWavesPerBlock = 4;

int clamp_wpr(int wpr) { return std::max(2, std::min(wpr, 8)); }

int lds_limit_bytes() { return 64 * 1024; }

// Kernel name of a launch target: the host-side handle of a __global__
// function carries the kernel's mangled name, which dladdr finds in the
// library's dynamic symbol table (no GPU needed); demangled, it is the name
// a rocprofv3 kernel trace shows.
void kernel_name(const void* handle, char* out, size_t len) {
  Dl_info di{};
  const char* mangled = (dladdr(handle, &di) && di.dli_sname) ? di.dli_sname : "?";
  int st = 0;
  char* dem = abi::__cxa_demangle(mangled, nullptr, nullptr, &st);
  std::snprintf(out, len, "%s", (st == 0 && dem) ? dem : mangled);
  std::free(dem);
}

// Dispatch stamps, one per device (dk_last_kernel_stamp): stamp + 1 of the
// last successful launch on that device, 0 for none since the last read.
constexpr int kStampDevices = 64;
std::atomic<int> g_stamps[kStampDevices];

// Launches one kernel on `stream` and reports a launch error as DK_ERR_HIP.
// With `info` set it launches nothing and records the kernel and its launch
// shape instead (dk_gemv_describe); the first launch of a call is recorded
// and every launch is counted.
struct Launch {
  hipStream_t stream;
  dk_launch_info* info = nullptr;

  // After a successful launch: records `stamp` as the dispatch stamp of the
  // device the launch went to (the stream's; the current device for the
  // null stream), not in describe mode. Returns rc.
  int stamp(int rc, int stamp) const {
    if (rc != DK_OK || info) return rc;
    int dev = 0;
    hipDevice_t sdev = 0;
    const bool ok = stream ? hipStreamGetDevice(stream, &sdev) == hipSuccess
                           : hipGetDevice(&dev) == hipSuccess;
    if (stream) dev = static_cast<int>(sdev);
    if (ok && dev >= 0 && dev < kStampDevices)
      g_stamps[dev].store(stamp + 1, std::memory_order_relaxed);
    return rc;
  }

  template <typename... KArgs, typename... Args>
  int operator()(const char* what, void (*kernel)(KArgs...), dim3 grid, dim3 block, size_t lds,
                 Args... args) const {
    if (info) {
      if (info->launches++ == 0) {
        kernel_name(reinterpret_cast<const void*>(kernel), info->kernel, sizeof(info->kernel));
        const unsigned g[3] = {grid.x, grid.y, grid.z}, b[3] = {block.x, block.y, block.z};
        for (int i = 0; i < 3; ++i) {
          info->grid[i] = g[i];
          info->block[i] = b[i];
        }
      }
      return DK_OK;
    }
    hipLaunchKernelGGL(kernel, grid, block, lds, stream, args...);
    return dk::check_launch(what);
  }
};

// The split-K kernel (gemv_v4_split): S waves per row, W waves per
// workgroup, R rows per wave, U chunks per lane per stage and slice, NB
// batch rows per stage, prefetch on or off. The activation stage (two
// buffers of NB S U 4 KiB) stays within 64 KiB.
struct SplitShape {
  int R, U, W, S, NB;
  bool pf;
};

template <int R, int U, int W, int S, int NB, bool PF>
int launch_split_t(const Launch& L, const uint4* p, const uint16_t* s, const uint4* x, uint16_t* y,
                   float* acc, int M, int K, int B) {
  constexpr int kRows = W / S * R;
  const dim3 grid((M + kRows - 1) / kRows, (B + NB - 1) / NB);
  return L("split-K launch", dk::gemv_v4_split<R, U, W, S, NB, PF>, grid, dim3(W * 64), 0, p, s, x,
           y, acc, M, K, B);
}

// acc: the reference's [B, M] fp32 buffer to receive the sums, or NULL.
int launch_split(const Launch& L, const uint4* p, const uint16_t* s, const uint4* x, uint16_t* y,
                 float* acc, int M, int K, int B, const SplitShape& sh) {
#define DK_SPLIT(r, u, w, k, nb, f)                                                          \
  if (sh.R == r && sh.U == u && sh.W == w && sh.S == k && sh.NB == nb && sh.pf == f)        \
    return launch_split_t<r, u, w, k, nb, f>(L, p, s, x, y, acc, M, K, B);
  DK_SPLIT(1, 2, 8, 1, 1, true) DK_SPLIT(1, 2, 8, 4, 1, false) DK_SPLIT(1, 4, 4, 2, 1, false)
  DK_SPLIT(1, 1, 4, 2, 1, true) DK_SPLIT(1, 2, 8, 4, 1, true) DK_SPLIT(1, 4, 4, 2, 1, true)
  DK_SPLIT(2, 2, 8, 4, 1, false) DK_SPLIT(1, 4, 8, 2, 1, false) DK_SPLIT(1, 2, 4, 2, 1, true)
  DK_SPLIT(1, 1, 8, 2, 1, true) DK_SPLIT(1, 1, 16, 2, 1, true) DK_SPLIT(2, 1, 4, 2, 1, false)
  DK_SPLIT(2, 2, 4, 2, 1, true) DK_SPLIT(2, 2, 8, 2, 1, false) DK_SPLIT(2, 1, 16, 2, 1, true)
  DK_SPLIT(2, 1, 16, 2, 1, false)
  DK_SPLIT(1, 2, 8, 1, 2, true) DK_SPLIT(1, 2, 8, 1, 4, true) DK_SPLIT(1, 1, 8, 2, 2, true)
  DK_SPLIT(1, 1, 8, 2, 4, true)
#undef DK_SPLIT
  return dk::set_error(DK_ERR_UNSUPPORTED, "split-K: no kernel for R%d U%d W%d S%d NB%d", sh.R,
                       sh.U, sh.W, sh.S, sh.NB);
}

// v4 launch plan. split_k caps the waves per row (S, a power of two, also at
// most K / 128 and 8). Set from a sweep of 62 shapes (R 1-2, U 1-4, W 4-16,
// S 2-8, prefetch on and off) at 24 shapes of M and K, timed back to back
// over cold weights, us per launch, the choice against the best:
//   M = K = 4096:         R1 U1 W8  S2 pf    3.62 (3.60)
//   M = 4096, K = 11008:  R1 U1 W16 S2 pf    6.10 (6.10)
//   M = 4096, K = 28672:  R2 U1 W16 S2 pf   11.53 (11.53)
//   M = 8192, K = 28672:  R2 U1 W16 S2      20.45 (20.45)
//   M = 8192, K = 8192:   R2 U2 W8  S2       7.84 (7.84)
//   M = 2048, K = 11008:  R1 U1 W16 S2 pf    4.64 (4.64)
//   M = 1024, K = 28672:  R2 U2 W8  S4       5.85 (5.85)
//   M = 512,  K = 28672:  R1 U2 W8  S4       4.60 (4.60)
//   M = 512,  K = 4096:   R1 U1 W4  S2 pf    2.16 (2.16)
// Eight waves per row (S = 8) were never the best (M = 512, K = 28672: 4.63
// against 4.58 for S = 4; M = K = 4096: 8.43 against 3.60 for S = 2); S = 1
// is the GEMV. Batches: S <= 2 with NB = 2 or 4 batch rows per stage.
SplitShape v4_plan(int M, int K, int B, int split_k) {
  const int G = K / DK_GROUP_SIZE;
  const int cap = std::max(1, std::min({split_k, G, 8}));
  const int s_max = cap >= 4 ? 4 : cap >= 2 ? 2 : 1;
  if (B > 1) {
    const int nb = B == 2 ? 2 : 4;
    return s_max == 1 ? SplitShape{1, 2, 8, 1, nb, true} : SplitShape{1, 1, 8, 2, nb, true};
  }
  if (s_max == 1) return {1, 2, 8, 1, 1, true};
  const bool tall = K >= 16384;
  const bool four = s_max >= 4;
  if (M <= 512) {
    if (tall) return four ? SplitShape{1, 2, 8, 4, 1, false} : SplitShape{1, 4, 4, 2, 1, false};
    if (K <= 4096) return {1, 1, 4, 2, 1, true};
    return four ? SplitShape{1, 2, 8, 4, 1, true} : SplitShape{1, 4, 4, 2, 1, true};
  }
  if (M <= 1024) {
    if (tall) return four ? SplitShape{2, 2, 8, 4, 1, false} : SplitShape{1, 4, 8, 2, 1, false};
    return K <= 8192 ? SplitShape{1, 2, 4, 2, 1, true} : SplitShape{1, 4, 4, 2, 1, true};
  }
  if (M <= 2048) return K <= 4096 ? SplitShape{1, 1, 8, 2, 1, true} : SplitShape{1, 1, 16, 2, 1, true};
  if (K <= 4096) return M <= 8192 ? SplitShape{1, 1, 8, 2, 1, true} : SplitShape{2, 1, 4, 2, 1, false};
  if (K <= 8192) return M <= 4096 ? SplitShape{2, 2, 4, 2, 1, true} : SplitShape{2, 2, 8, 2, 1, false};
  if (K <= 12288) return {1, 1, 16, 2, 1, true};
  return M <= 4096 ? SplitShape{2, 1, 16, 2, 1, true} : SplitShape{2, 1, 16, 2, 1, false};
}

int launch_v4(const Launch& L, const uint4* p, const uint16_t* s, const uint4* x, uint16_t* y,
              float* acc, int M, int K, int B, int split_k) {
  return launch_split(L, p, s, x, y, acc, M, K, B, v4_plan(M, K, B, split_k));
}

// One batch row at the shapes where the split-K kernel beats gemv_v5_lds by
// 5% or more in the same sweep (us, split-K against gemv_v5_lds):
//   M = 4096, K = 11008:  6.12 (6.44)     M = 4096, K = 14336:  7.64 (8.19)
//   M = 4096, K = 28672: 11.53 (12.67)    M = 5120, K = 8192:   5.94 (6.28)
//   M = 8192, K = 8192:   7.84 (8.13)     M = 1024, K = 28672:  5.85 (6.74)
//   M = 512,  K = 28672:  4.60 (6.21)     M = 512,  K = 8320:   2.91 (3.05)
//   M = 512,  K = 4096:   2.16 (2.28)
// Elsewhere it is level or slower (M = K = 4096: 3.62 against 3.54; M =
// 11008, K = 5120: 9.34 against 8.48; M = 1024, K = 11008: 3.63 against
// 3.31).
bool v5_takes_split(int M, int K, SplitShape* sh) {
  if (M <= 512 && K > 2048) {
    *sh = K >= 16384 ? SplitShape{1, 2, 8, 4, 1, false}
          : K <= 4096 ? SplitShape{1, 1, 4, 2, 1, true}
                      : SplitShape{1, 2, 8, 4, 1, true};
    return true;
  }
  if (M <= 1024 && K >= 16384) {
    *sh = {2, 2, 8, 4, 1, false};
    return true;
  }
  if (M > 3072 && M <= 4096 && K > 8192) {
    *sh = K <= 12288 ? SplitShape{1, 1, 16, 2, 1, true} : SplitShape{2, 1, 16, 2, 1, true};
    return true;
  }
  if (M > 4096 && M <= 8192 && K == 8192) {
    *sh = {2, 2, 8, 2, 1, false};
    return true;
  }
  return false;
}

// One activation row: the streaming kernel with activations shared through
// LDS (R rows per wave, U 16-byte chunks per lane per stage, W waves per
// workgroup, next stage prefetched or not). Timed on MI355X as the bench
// times it: a HIP graph of back-to-back steps over torch-allocated weight
// copies (> 640 MB, cold), us per step, against the earlier form of the
// kernel that loaded the activations per wave into registers ("registers":
// R2 U2, or R4 U1 at the 70B shapes, two waves per workgroup):
//   M = K = 4096:         R1 U2 W8 prefetch 3.59 (R2 U2 W4 3.69; registers 3.73)
//   M = 11008, K = 4096:  R2 U2 W4 5.83 (W8 5.72, prefetch 5.75; registers 6.32)
//   M = 4096, K = 11008:  R1 U2 W16 prefetch 6.07 (no prefetch 6.49; registers 7.08)
//   M = 28672, K = 8192:  R2 U2 W4 20.73 (prefetch 22.60; registers 23.04)
//   M = 8192, K = 28672:  R2 U1 W16 prefetch 20.17 (no prefetch 19.79; registers 22.24)
//   M = 8192, K = 3584:   R1 U2 W8 prefetch 4.40 (registers 5.23)
//   M = 8192, K = 8192:   R2 U1 W16 prefetch 7.73 (R1 U2 W8 prefetch 8.15; registers 8.47)
//   M = 4096, K = 2048:   R1 U1 W16 prefetch 2.72 (R1 U2 W8 prefetch 3.27; registers 3.46)
//   M = K = 28672:        R2 U1 W8 64.65 (registers 75.82)
// Over 19 shapes (M and K from 2048 to 28672) the choice below is within 1%
// of the best of 18 variants on average and 6.5% at worst. Prefetching pays
// when rows are few (few waves per SIMD to hide a stage's latency) and costs
// occupancy when they are many; 16-wave workgroups share each activation
// load among more rows when stages are many.
// Up to 3072 rows (tensor-parallel shards) the grid is the limit: four-wave
// workgroups, and stages of U = 4 or 6 chunks per lane so that a row of up
// to 12288 weights is one stage (each wave waits for one round of loads),
// against the rule for larger M (one row per wave, U = 2 or 1, W = 8 or 16):
//   M = 512,  K = 8320:  R1 U6 W4 prefetch 3.03 (5.09)
//   M = 1024, K = 8192:  R1 U4 W4 prefetch 2.82 (3.83)
//   M = 1280, K = 8192:  R1 U4 W4 prefetch 3.20 (3.92)
//   M = 2048, K = 11008: R1 U6 W4 prefetch 4.34 (5.37)
//   M = 3072, K = 8192:  R1 U4 W4 prefetch 4.23 (4.74)
//   M = 2048, K = 16384: R1 U4 W8 prefetch 5.63 (6.79)
//   M = 1024, K = 28672: R1 U4 W4 prefetch 6.50 (9.53)
//   M = 512,  K = 4096:  R1 U2 W4 prefetch 2.28 (2.56)
// (the best of 48 variants, U from 2 to 6, at each of these shapes but
// M = 1024, K = 28672, where R1 U3 W4 is 0.3% faster).
// At M = 4096 the wide stages lose (M = 4096, K = 11008: R1 U6 W4 7.26
// against R1 U2 W16 prefetch 6.04).
// Rows of 4097-8191 weights above 3072 rows: stages of 2048 weights (U = 1,
// 16 waves) leave less of the last stage empty than stages of 4096 (R1 U2
// W8, the rule for K <= 4096), 10-22% faster (us):
//   M = 3328, K = 5120: 4.24 (4.85)     M = 4096, K = 5120: 4.32 (4.98)
//   M = 4096, K = 6144: 4.35 (5.02)     M = 4608, K = 6144: 5.25 (5.90)
//   M = 5120, K = 5120: 5.30 (5.89)     M = 6144, K = 6144: 5.43 (6.22)
//   M = 8192, K = 5120: 5.71 (7.27)     M = 8192, K = 6144: 5.88 (7.53)
// and rows of 8192 up to 5120 rows take one stage of U = 4 per row:
// M = 3584: 4.83 (4.89); M = 4096: 5.02 (5.16); M = 5120: 6.11 (6.43).
// Above 8192 rows the same rows take two rows per wave with stages of 2048
// weights (R2 U1 W8 prefetch): M = 11008, K = 5120: 7.80 (8.73 for R2 U2 W4);
// M = 13824, K = 5120: 9.27 (9.85).
template <int R, int U, int W, bool kPrefetch, typename Layout, int kStamp, int NB = 1>
int launch_lds_t(const Launch& L, const uint4* p, const uint16_t* s, const uint4* x, uint16_t* y,
                 int M, int K, int B = 1) {
  dim3 grid((M + W * R - 1) / (W * R), (B + NB - 1) / NB);
  return L("v5 launch", dk::gemv_v5_lds<R, U, W, NB, kPrefetch, Layout, kStamp>, grid, dim3(W * 64),
           0, p, s, x, y, M, K, B);
}

template <typename Layout, int kStamp>
int launch_lds(const Launch& L, const uint4* p, const uint16_t* s, const uint4* x, uint16_t* y,
               int M, int K) {
  SplitShape sh;
  if (std::is_same<Layout, dk::LayoutLogical>::value && v5_takes_split(M, K, &sh))
    return launch_split(L, p, s, x, y, nullptr, M, K, 1, sh);
  if (K <= 2048) return launch_lds_t<1, 1, 16, true, Layout, kStamp>(L, p, s, x, y, M, K);
  if (M <= 3072) {
    if (K <= 4096) return launch_lds_t<1, 2, 4, true, Layout, kStamp>(L, p, s, x, y, M, K);
    if (K <= 8192) return launch_lds_t<1, 4, 4, true, Layout, kStamp>(L, p, s, x, y, M, K);
    if (K <= 12288) return launch_lds_t<1, 6, 4, true, Layout, kStamp>(L, p, s, x, y, M, K);
    if (M <= 1024) return launch_lds_t<1, 4, 4, true, Layout, kStamp>(L, p, s, x, y, M, K);
    return launch_lds_t<1, 4, 8, true, Layout, kStamp>(L, p, s, x, y, M, K);
  }
  if (M <= 8192 && K > 4096 && K < 8192)
    return launch_lds_t<1, 1, 16, true, Layout, kStamp>(L, p, s, x, y, M, K);
  if (M <= 5120 && K == 8192) return launch_lds_t<1, 4, 4, true, Layout, kStamp>(L, p, s, x, y, M, K);
  if (M > 8192) {
    if (K > 4096 && K < 8192) return launch_lds_t<2, 1, 8, true, Layout, kStamp>(L, p, s, x, y, M, K);
    if (K <= 8192) return launch_lds_t<2, 2, 4, false, Layout, kStamp>(L, p, s, x, y, M, K);
    return launch_lds_t<2, 1, 8, false, Layout, kStamp>(L, p, s, x, y, M, K);
  }
  if (K > 8192 && M <= 4096) return launch_lds_t<1, 2, 16, true, Layout, kStamp>(L, p, s, x, y, M, K);
  if (K >= 8192 && M > 4096) return launch_lds_t<2, 1, 16, true, Layout, kStamp>(L, p, s, x, y, M, K);
  return launch_lds_t<1, 2, 8, true, Layout, kStamp>(L, p, s, x, y, M, K);
}

// Batches: the same LDS kernel with NB batch rows per stage (grid.y covers
// the batch in tiles of NB rows). Timed as above, us per launch, the choice
// below against the previous rule (NB = 2 tiles for B = 2, NB = 4 tiles
// otherwise, one shape per M range):
//                        B = 2           B = 3           B = 4
//   M = 512, K = 8320:   4.38 (5.12)     4.40 (5.79)     4.41 (7.39)
//   M = 1024, K = 11008: 4.58 (5.29)     5.22 (5.95)     5.31 (7.50)
//   M = 2048, K = 16384: 7.12 (7.11)     7.86 (7.89)     8.64 (10.11)
//   M = K = 4096:        3.94 (3.93)     4.45 (4.71)     4.95 (5.19)
//   M = 4096, K = 11008: 7.49 (7.42)     8.62 (9.93)     10.00 (11.12)
//   M = 4096, K = 28672: 14.64 (15.47)   17.61 (19.09)   20.61 (23.75)
//   M = 6144, K = 8192:  8.23 (8.69)     10.01 (12.05)   11.65 (12.18)
//   M = 11008, K = 4096: 6.80 (7.20)     8.51 (9.23)     9.44 (9.52)
//   M = 8192, K = 28672: 24.30 (25.75)   30.00 (36.80)   34.20 (37.99)
//   M = 28672, K = 8192: 25.65 (26.32)   32.26 (34.13)   35.62 (35.47)
// B = 5 and 6 run two tiles of three rows (the previous rule's four-row
// tiles left three rows of the second empty at B = 5): M = 1024, K = 11008
// 5.97 (7.52); M = 4096, K = 14336 14.52 (26.59). Over 18 shapes (M from 512
// to 28672, K from 3584 to 28672) the choice is 2-3% from the best of 72
// variants (R, U, W, prefetch, NB) per batch size on average and 8-17% at
// worst. What decides is the number of workgroups: one per CU (256) with as
// many rows and batch rows in each as that allows shares every activation
// load most widely, so small M takes narrow workgroups and splits the batch
// into more tiles (NB = 2 at B = 4 for M <= 1024: 4.41 against 7.39 us at
// M = 512), and large M takes wide ones with every batch row in one tile.
// Up to 2048 rows of 4097-8192 weights, stages of U = 4 (one per row) in
// two-row tiles: M = 1024, K = 8192: B = 2 3.19 (3.98), B = 3 3.72 (4.45),
// B = 4 3.80 (4.56); M = 2048, K = 8192, B = 2: 4.15 (4.91); M = 768,
// K = 8192, B = 3: 3.61 (4.37); M = 512, K = 8192, B = 4: 3.12 (3.85).
#define DK_BATCH(R, U, W, PF, NB) \
  launch_lds_t<R, U, W, PF, Layout, kStamp, NB>(L, p, s, x, y, M, K, B)
template <typename Layout = dk::LayoutLogical, int kStamp = Layout::kStamp>
int launch_v5(const Launch& L, const uint4* p, const uint16_t* s, const uint4* x, uint16_t* y, int M,
              int K, int B) {
  if (B == 1) return launch_lds<Layout, kStamp>(L, p, s, x, y, M, K);
  const bool long_rows = K > 8192;
  // Few rows with one-stage rows of up to 8192 weights (U = 4).
  const bool one_wide_stage = K > 4096 && K <= 8192;
  // Above 2048 rows, rows of 4097-8191 weights take stages of 2048 weights
  // (us, against the rule for K <= 4096 or K = 8192 in brackets):
  //   B = 2: M = 4096, K = 6144 4.95 (6.07); M = 5120, K = 5120 5.79 (6.56);
  //          M = 8192, K = 6144 7.26 (7.34); M = 11008, K = 5120 9.32 (11.60);
  //          M = 13824, K = 5120 11.78 (14.24)
  //   B = 4: M = 4096, K = 6144 6.58 (8.32); M = 5120, K = 5120 8.99 (11.31);
  //          M = 8192, K = 6144 9.62 (12.05); M = 11008, K = 5120 12.79 (13.32)
  const bool mid_rows = M > 2048 && K > 4096 && K < 8192;
  if (mid_rows && B == 2) {
    if (M <= 4096) return DK_BATCH(1, 1, 16, true, 2);
    if (M <= 6144) return DK_BATCH(1, 1, 8, true, 2);
    if (M <= 8192) return DK_BATCH(1, 1, 16, true, 2);
    return DK_BATCH(2, 1, 8, true, 2);
  }
  if (mid_rows && B == 3) return DK_BATCH(2, 1, 8, true, 3);
  if (mid_rows && B == 4) return DK_BATCH(2, 1, 8, true, 4);
  if (B == 2) {
    if (one_wide_stage && M <= 1024) return DK_BATCH(1, 4, 4, true, 2);
    if (one_wide_stage && M <= 2048) return DK_BATCH(2, 4, 4, true, 2);
    if (M <= 1024) return DK_BATCH(1, 2, 4, true, 2);
    if (M <= 2048 || (M <= 4096 && K <= 12288)) return DK_BATCH(1, 2, 8, true, 2);
    if (M <= 4096) return DK_BATCH(2, 2, 8, true, 2);
    if (M > 8192) return DK_BATCH(2, 2, 8, false, 2);
    return K <= 4096 ? DK_BATCH(2, 2, 4, true, 2) : DK_BATCH(2, 1, 16, false, 2);
  }
  if ((B == 3 || B == 4) && one_wide_stage && M <= 1024)
    return M <= 512 ? DK_BATCH(1, 4, 4, true, 2) : DK_BATCH(1, 4, 8, true, 2);
  if (B == 3) {
    if (M <= 512) return DK_BATCH(1, 2, 4, true, 2);
    if (M <= 1024) return DK_BATCH(1, 2, 4, true, 3);
    if (M <= 2048) return DK_BATCH(1, 2, 8, true, 3);
    if (M <= 4096) return long_rows ? DK_BATCH(1, 2, 16, true, 3) : DK_BATCH(1, 2, 8, true, 3);
    return DK_BATCH(2, 2, 8, false, 3);
  }
  if (B == 4) {
    if (M <= 512) return DK_BATCH(1, 2, 4, true, 2);
    if (M <= 1024) return DK_BATCH(1, 2, 8, true, 2);
    if (M <= 2048) return DK_BATCH(2, 2, 8, true, 2);
    if (M <= 4096) return long_rows ? DK_BATCH(2, 2, 8, true, 4) : DK_BATCH(1, 2, 8, true, 4);
    return M > 8192 ? DK_BATCH(2, 1, 8, false, 4) : DK_BATCH(2, 2, 8, false, 4);
  }
  if (B <= 6) {
    if (M <= 512) return DK_BATCH(1, 2, 4, true, 3);
    if (M <= 1024) return DK_BATCH(1, 2, 8, true, 3);
    if (M <= 2048) return DK_BATCH(2, 2, 8, true, 3);
    if (M <= 4096 || K > 4096) return DK_BATCH(2, 1, 16, true, 3);
    return DK_BATCH(2, 2, 8, false, 3);
  }
  // Seven or eight rows of 4097-8191 weights at 513-2048 rows: stages of
  // 2048 weights in two four-row tiles (us, B = 8): M = 2048, K = 5120 6.26
  // (7.36); M = 1536, K = 6144 6.19 (7.25); M = 1024, K = 6144 4.90 (5.52);
  // level at M = 400, K = 5120 (5.07 against 5.02).
  if (B <= 8 && M > 512 && M <= 2048 && K > 4096 && K < 8192)
    return M <= 1024 ? DK_BATCH(1, 1, 8, true, 4) : DK_BATCH(1, 1, 16, true, 4);
  if (M <= 1024) return DK_BATCH(1, 2, 8, true, 2);
  if (M <= 2048) return DK_BATCH(2, 2, 8, true, 4);
  if (M <= 4096) return DK_BATCH(2, 1, 16, true, 4);
  return M > 8192 ? DK_BATCH(2, 1, 8, false, 4) : DK_BATCH(2, 2, 8, false, 4);
}
#undef DK_BATCH

// Batches that the MFMA tiles take on the fused gate/up step. Tiles against
// the streaming kernel's batch tiles in brackets (us per launch, both
// matrices; 8 waves, blocks of two groups, chosen over 4 or 16 waves with
// blocks of two and 8 waves with blocks of four, 2-40% slower at B = 4, 8
// and 16 on five shapes; * marks the streaming kernel where it is chosen):
//                        B = 3           B = 4           B = 5           B = 8           B = 16
//   I = 11008, H = 4096: 13.62 (14.92)   13.77 (19.25)   13.78 (24.31)   14.62 (31.51)   18.72 (58.31)
//   I = 3584,  H = 8192: 11.07 (10.74*)  11.15 (12.64)   11.39 (18.88)   11.96 (23.55)   13.89 (45.13)
//   I = 28672, H = 8192: 50.73 (59.49)   52.05 (70.56)   52.96 (108.97)  59.11 (129.76)  76.80 (256.50)
//   I = 2752,  H = 4096: 6.62 (7.03)     6.66 (8.34)     6.75 (11.62)    7.20 (15.39)    8.26 (22.66)
//   I = 1376,  H = 4096: 6.37 (4.66*)    6.42 (5.28*)    6.42 (5.53*)
// Two batch rows stream everywhere (I = 11008: 13.38 against 12.56); three
// take the tiles at I = 3584, H = 8192 as well (9.48 against 11.19 for the
// streaming kernel in a later sweep).
// Up to 2048 rows, where the scales pair, the double-buffered tiles
// (gate_up_silu_tiles_pf, I / 16 workgroups: their time barely depends on I
// or B) take over from the streaming kernel once B I exceeds 8192; at most
// 512 rows the streaming kernel stays to 16 batch rows. Against the
// streaming kernel (us, H = 4096 / 8192):
//   I = 1024, B = 8: 5.71 (5.33) / 8.77 (8.25); B = 12: 5.90 (7.48) / 9.26 (12.42)
//   I = 1376, B = 5: 5.77 (5.56) / 8.89 (9.37); B = 8: 5.77 (7.33) / 8.90 (12.05)
//   I = 1792, B = 5: 5.80 (6.75) / 8.92 (11.96); B = 8: 5.84 (9.01) / 9.02 (15.50)
//   I = 2048, B = 5: 5.88 (7.00) / 8.94 (12.42); B = 8: 5.87 (9.33) / 9.03 (15.71)
//   I = 512, B = 16: 6.03 (5.40) / 9.89 (8.31)
// (3-4 batch rows stream at every I up to 2048: I = 2048, B = 4 5.73 against
// 5.37 at H = 4096.) Where the scales do not pair the earlier rule holds.
bool gate_up_tiles(int I, int H, int B, bool pairs) {
  (void)H;
  if (B <= 2) return false;
  if (pairs && I > 512 && I <= 2048 && B <= 16) return (long long)B * I > 8192;
  return !((B <= 8 && I <= 2048) || (B <= 16 && I <= 1024));
}

// Fused gate/up, R rows of each matrix per wave, on the LDS stage loop (U
// chunks per stage, W waves per workgroup, next stage prefetched or not, NB
// batch rows per stage). Timed on MI355X back-to-back over cold weights (us
// per launch for both matrices), against the fused kernel with activations
// in registers (two waves per workgroup, R2 U1, NB2 tiles for batches):
//   I = 11008, H = 4096:  R1 U2 W4 9.17 (prefetch 9.57, W8 9.75; registers 10.25)
//                         B = 2: R1 U2 W4 prefetch 12.44 (registers 13.71)
//                         B = 4: R1 U1 W8 NB4 19.56 (registers 22.65)
//   I = 14336, H = 4096:  R1 U2 W4 11.88 (prefetch 11.65; registers 12.43)
//   I = 3584,  H = 8192:  R1 U1 W16 prefetch 7.37 (W8 7.45; registers 7.82)
//                         B = 2: 8.82 (registers 9.89); B = 4: NB4 12.71 (registers 17.20)
//   I = 14336, H = 8192:  R1 U2 W8 20.90 (W4 21.43; registers 23.27)
//   I = 28672, H = 8192:  R1 U2 W8 38.91 (R2 U1 W8 38.82; registers 40.17)
//                         B = 2: R2 U1 W4 48.56 (registers 55.51)
//                         B = 4: R1 U1 W8 NB4 74.52 (registers 107.87)
//   I = 4096,  H = 4096:  R1 U2 W4 prefetch 5.02 (registers 5.29)
template <int R, int U, int W, bool kPrefetch, int NB = 1>
int launch_gate_up_lds_t(const Launch& L, const uint4* g, const uint16_t* gs, const uint4* u,
                         const uint16_t* us, const uint4* x, uint16_t* h, int I, int H, int B = 1) {
  dim3 grid((I + W * R - 1) / (W * R), (B + NB - 1) / NB);
  return L("gate/up launch", dk::gate_up_silu_lds<R, U, W, NB, kPrefetch>, grid, dim3(W * 64), 0, g,
           gs, u, us, x, I, H, B, h);
}

// Batches: tiles of two batch rows at B = 2, three at B = 3, 5 and 6, four
// otherwise, as for the GEMV. Timed as above (us per launch), against the
// previous rule (NB = 4 tiles from B = 3 on, no separate small-I case):
//                        B = 2           B = 3           B = 4
//   I = 1376, H = 4096:  4.09 (5.40)     4.70 (7.82)     5.26 (8.09)
//   I = 1792, H = 8192:  6.13 (8.15)     7.11 (11.86)    8.30 (12.21)
//   I = 3584, H = 8192:  8.78 (8.94)     10.65 (12.43)   12.70 (12.75)
//   I = 11008, H = 4096: 12.04 (12.30)   14.95 (17.25)   17.88 (18.64)
//   I = 14336, H = 4096: 15.00 (15.61)   17.33 (20.29)   20.45 (21.06)
//   I = 28672, H = 8192: 47.02 (47.29)   58.23 (66.36)   66.48 (69.62)
// Within 2.5% of the best of 72 variants (R, U, W, prefetch, NB) at every
// one of these shapes but I = 1376, B = 4 (8%: two tiles of two rows do
// better there). Small I takes narrow workgroups (W = 4) so that the grid
// still covers the chip. One batch row with I <= 2048 and H of 4097-8192
// takes one stage of U = 4 per row: I = 1024, H = 8192: 3.72 (6.12);
// I = 1792: 4.87 (6.40); I = 2048: 5.05 (6.47); at I = 3584 it is no better
// than R1 U1 W16 (7.73 against 7.51).
#define DK_GATE_UP(R, U, W, PF, NB) \
  launch_gate_up_lds_t<R, U, W, PF, NB>(L, g, gs, u, us, x, h, I, H, B)
int launch_gate_up(const Launch& L, const uint4* g, const uint16_t* gs, const uint4* u,
                   const uint16_t* us, const uint4* x, uint16_t* h, int I, int H, int B) {
  const bool pairs = (H / DK_GROUP_SIZE) % 2 == 0 && aligned(gs, 4) && aligned(us, 4);
  if (gate_up_tiles(I, H, B, pairs)) {
    const dim3 grid((I + 15) / 16, (B + dk::kReuseBatch - 1) / dk::kReuseBatch);
    // From 8 batch rows, both tiles' operands staged in LDS (as the GEMV's
    // gemv_reuse_lds), 8 waves up to I = 4096 and 16 batch rows, else 4
    // (us, against the tiles that load the operands directly):
    //                        B = 8           B = 16          B = 32
    //   I = 11008, H = 4096: 13.91 (14.50)   16.05 (19.06)   27.97 (34.47)
    //   I = 14336, H = 4096: 17.98 (17.72)   20.36 (24.09)   34.24 (43.83)
    //   I = 3584,  H = 8192: 10.66 (11.70)   11.91 (13.97)   19.53 (24.65)
    //   I = 2752,  H = 4096: 6.64 (7.01)     7.08 (8.50)     11.40 (13.78)
    //   I = 28672, H = 8192: 57.23 (59.11)   66.36 (80.54)   127.57 (158.15)
    // Up to 4 batch rows the direct tiles stay (I = 11008, H = 4096, B = 4:
    // 12.25 against 12.57; I = 28672, B = 3: 47.68 against 50.50). Up to
    // I = 4096 at 9-16 batch rows, double buffered with 4 waves (the GEMV's
    // gemv_reuse_pf; us, against the best single-buffered kernel): I = 3584,
    // H = 8192, B = 16 11.28 (11.98); I = 2752, H = 4096, B = 16 6.85
    // (7.20). With more tiles than CUs they lose to the single-buffered 4
    // waves, which fit three workgroups per CU (I = 11008, H = 4096, B = 16:
    // 17.76 against 15.67).
    if (pairs && I <= 4096 && B >= 9 && B <= 16)
      return L("gate/up launch", dk::gate_up_silu_tiles_pf<4>, grid, dim3(4 * 64), 0, g, gs, u, us,
               x, I, H, B, h);
    // Below 9 batch rows, with four x loads per block (the x buffers then
    // hold 8 rows: two workgroups per CU): I = 3584, H = 8192, B = 3 9.08
    // (9.40), B = 8 9.63 (10.34); I = 28672, H = 8192, B = 3 45.93 (46.95),
    // B = 8 51.42 (56.29); I = 11008, H = 4096, B = 8 12.93 (13.51). From
    // 4097 to 16384 rows the direct tiles keep 3-4 batch rows (I = 11008,
    // B = 3: 11.97 against 12.31).
    if (pairs && B <= 8 && (I <= 4096 || I > 16384 || B >= 5))
      return L("gate/up launch", dk::gate_up_silu_tiles_pf<4, 4>, grid, dim3(4 * 64), 0, g, gs, u,
               us, x, I, H, B, h);
    if (B >= 8) {
      if (I <= 4096 && B <= 16)
        return pairs ? L("gate/up launch", dk::gate_up_silu_tiles_lds<8, true>, grid, dim3(8 * 64),
                         0, g, gs, u, us, x, I, H, B, h)
                     : L("gate/up launch", dk::gate_up_silu_tiles_lds<8, false>, grid,
                         dim3(8 * 64), 0, g, gs, u, us, x, I, H, B, h);
      return pairs ? L("gate/up launch", dk::gate_up_silu_tiles_lds<4, true>, grid, dim3(4 * 64), 0,
                       g, gs, u, us, x, I, H, B, h)
                   : L("gate/up launch", dk::gate_up_silu_tiles_lds<4, false>, grid, dim3(4 * 64),
                       0, g, gs, u, us, x, I, H, B, h);
    }
    // Paired scale loads up to 8 batch rows, as for the GEMV: I = 11008,
    // H = 4096, B = 4: 12.28 against 13.67 us.
    if (pairs)
      return L("gate/up launch", dk::gate_up_silu_tiles<8, 2, true>, grid, dim3(8 * 64), 0, g, gs, u,
               us, x, I, H, B, h);
    return L("gate/up launch", dk::gate_up_silu_tiles<8, 2, false>, grid, dim3(8 * 64), 0, g, gs, u,
             us, x, I, H, B, h);
  }
  if (B == 1) {
    // Few rows of up to 8192 weights: one stage of U = 4 per row.
    if (I <= 2048 && H > 4096 && H <= 8192) return DK_GATE_UP(1, 4, 4, true, 1);
    if (I <= 4096) return H > 4096 ? DK_GATE_UP(1, 1, 16, true, 1) : DK_GATE_UP(1, 2, 4, true, 1);
    // Rows of 4097-8191 weights: stages of 2048 (us, against R1 U2 W8):
    // I = 11008, H = 5120: 12.80 (15.34); I = 13824, H = 5120: 14.99
    // (17.38); I = 14336, H = 6144: 16.47 (18.31); I = 8192, H = 6144: 10.35
    // (11.69).
    if (H > 4096 && H < 8192) return DK_GATE_UP(1, 1, 8, true, 1);
    return H <= 4096 ? DK_GATE_UP(1, 2, 4, false, 1) : DK_GATE_UP(1, 2, 8, false, 1);
  }
  if (B == 2) {
    if (I <= 2048) return DK_GATE_UP(1, 2, 4, true, 2);
    if (I <= 4096) return DK_GATE_UP(1, 1, 16, true, 2);
    return H <= 4096 ? DK_GATE_UP(1, 2, 8, false, 2) : DK_GATE_UP(2, 1, 4, false, 2);
  }
  if (B == 3 || B == 5 || B == 6) {
    if (I <= 2048) return DK_GATE_UP(1, 2, 4, true, 3);
    if (I <= 4096) return DK_GATE_UP(1, 1, 16, true, 3);
    return DK_GATE_UP(2, 2, 4, false, 3);
  }
  if (I <= 2048) return DK_GATE_UP(1, 2, 4, true, 4);
  if (I <= 4096) return DK_GATE_UP(1, 1, 16, true, 4);
  return DK_GATE_UP(2, 1, 4, false, 4);
}
#undef DK_GATE_UP

// The reuse path's tiles that load the MFMA operands directly (gemv_reuse:
// KS waves per 16-row tile, RT tiles per wave, blocks of SG groups, weights
// through wave-private LDS, x in the MFMA B layout straight from memory).
// They take the shapes where the LDS-staged tiles (launch_reuse_lds below)
// measured slower: M > 8192 with rows longer than 4096 weights up to 8 batch
// rows, and rows of up to 4096 weights at 2049-4096 rows up to 5. Measured
// when they ran every tile shape (us per launch, against the streaming
// kernel's batch tiles in brackets, * where those were chosen):
//                        B = 2          B = 3          B = 4          B = 5    B = 8    B = 16
//   M = 28672, K = 8192: 29.08 (25.69*) 29.59 (33.42)  30.31 (36.87)  30.29    33.65    44.04
//   M = 8192, K = 28672: 29.65 (24.58*) 29.40 (30.99)  29.68 (35.14)  30.24    32.76    40.91
//   M = K = 4096:        4.66 (3.93*)   4.73 (4.44*)   4.82 (4.95)    4.82     5.23     6.82
// The tiles cost about the same from one batch row to five (16 MFMA batch
// columns); two tiles per wave share each activation load once there are
// enough tiles for the chip (M > 4096). The weights come through LDS in
// 128-256 contiguous bytes per row (8-20% faster than loading the MFMA
// layout directly at M = 11008 or K = 28672).
template <int KS, int RT, int SG>
int launch_reuse(const Launch& L, const uint4* p, const uint16_t* s, const uint4* x, uint16_t* y,
                 int M, int K, int B) {
  const dim3 grid((M + 16 * RT - 1) / (16 * RT), (B + dk::kReuseBatch - 1) / dk::kReuseBatch);
  // Paired scale loads (fewer registers: 92 against 98 for two tiles per
  // wave) need an even number of groups per row and 4-byte aligned scales
  // (the API asks for 2). They pay up to 8 batch rows (us, against single
  // scale loads): M = 8192, K = 28672, B = 4
  // 26.04 (29.73); M = 8192, K = 8192, B = 4 9.84 (11.32); M = K = 4096,
  // B = 4 4.70 (4.83); level at B = 8; at B = 16 they cost 0-5%
  // (M = 28672, K = 8192: 46.03 against 43.93).
  if constexpr (SG == 2) {
    if ((K / DK_GROUP_SIZE) % 2 == 0 && aligned(s, 4) && B <= 8)
      return L("reuse launch", dk::gemv_reuse<KS, RT, SG, true>, grid, dim3(KS * 64), 0, p, s, x, y,
               M, K, B);
  }
  return L("reuse launch", dk::gemv_reuse<KS, RT, SG, false>, grid, dim3(KS * 64), 0, p, s, x, y, M,
           K, B);
}

template <int KS, int RT, int SG = 2>
int launch_reuse_lds(const Launch& L, const uint4* p, const uint16_t* s, const uint4* x,
                     uint16_t* y, int M, int K, int B) {
  const dim3 grid((M + 16 * RT - 1) / (16 * RT), (B + dk::kReuseBatch - 1) / dk::kReuseBatch);
  if ((K / DK_GROUP_SIZE) % 2 == 0 && aligned(s, 4))
    return L("reuse launch", dk::gemv_reuse_lds<KS, RT, true, SG>, grid, dim3(KS * 64), 0, p, s, x,
             y, M, K, B);
  return L("reuse launch", dk::gemv_reuse_lds<KS, RT, false, SG>, grid, dim3(KS * 64), 0, p, s, x,
           y, M, K, B);
}

template <int KS, int RT, int XL>
int launch_reuse_pf(const Launch& L, const uint4* p, const uint16_t* s, const uint4* x, uint16_t* y,
                    int M, int K, int B) {
  // XL < 8 stages only batch rows 0 .. 2 XL - 1 of one batch tile.
  if (XL < 8 && B > 2 * XL)
    return fail(DK_ERR_UNSUPPORTED, "internal: %d x loads per block cannot serve %d batch rows", XL,
                B);
  const dim3 grid((M + 16 * RT - 1) / (16 * RT), (B + dk::kReuseBatch - 1) / dk::kReuseBatch);
  return L("reuse launch", dk::gemv_reuse_pf<KS, RT, XL>, grid, dim3(KS * 64), 0, p, s, x, y, M, K,
           B);
}

// The many-batch tiles (gemv_reuse_pfb): RT row tiles and NBT batch tiles
// per workgroup of KS waves; KS = 0: not these tiles.
struct PfbShape {
  int ks = 0, rt = 0, nbt = 0;
};

template <int KS, int RT, int NBT>
int launch_reuse_pfb(const Launch& L, const uint4* p, const uint16_t* s, const uint4* x,
                     uint16_t* y, int M, int K, int B) {
  const dim3 grid((M + 16 * RT - 1) / (16 * RT), (B + 16 * NBT - 1) / (16 * NBT));
  return L("reuse launch", dk::gemv_reuse_pfb<KS, RT, NBT>, grid, dim3(KS * 64), 0, p, s, x, y,
           M, K, B);
}

// Above 16 batch rows (where the groups pair), the many-batch tiles. Of the
// shapes RT x NBT = 1 x 2, 2 x 2, 4 x 2, 4 x 4 (NBT = 4 only from three batch
// tiles), in order of reuse, the first whose grid is one round of 144-256
// workgroups (one per CU: four waves, 82-139 KiB of LDS); below 144 the one
// before it; where none reaches one round, 4 x 4 (or 4 x 2 up to 32 batch
// rows) with two waves when its grid is at most 512, so that two
// workgroups per CU make one round. Up to 32 batch rows only with RT >= 2:
// there the two batch columns of the single-tile kernels beat RT = 1.
// From sweeps of 14 shapes (KS, RT, NBT) at 12 (M, K) and B = 24-256, us,
// the chosen shape against the earlier dispatch (gemv_reuse_lds or
// gemv_reuse_pf, one workgroup per batch tile of 16):
//                        B = 48           B = 128          B = 256
//   M = K = 4096:        8.36 (11.36)     13.03 (21.06)    20.47 (39.94)
//   M = 4096, K = 11008: 17.89 (24.46)    29.38 (46.57)    46.98 (93.26)
//   M = 11008, K = 4096: 20.82 (21.57)    38.11 (45.44)    61.24 (87.96)
//   M = 2048, K = 8192:  10.75 (13.27)    13.85 (24.54)    22.11 (48.48)
//   M = 8192, K = 8192:  23.61 (28.43)    37.58 (68.98)    66.34 (140.76)
//   M = 3584, K = 8192:  14.12 (18.33)    22.32 (34.93)    36.16 (62.53)
//   M = 1024, K = 4096:  (4.97: earlier)  6.33 (8.67)      8.01 (15.66)
//   M = 28672, K = 8192: 69.32 (97.50)    129.53 (248.57)  250.81 (489.97)
// At 24-32 batch rows: M = 8192, K = 8192 16.07 (20.65); M = 6144, K =
// 8192 15.34 (18.66); M = 11008, K = 4096 13.96 (14.81); M = 28672, K =
// 8192 46.94 (66.60); M = K = 4096 keeps the earlier tiles (6.42 against
// 7.02 for RT = 1). Slower than the earlier dispatch at one shape of those
// swept: M = K = 5120, B = 48 (16.46 against 12.92; B = 64: 16.56 against
// 17.66).
PfbShape reuse_pfb_shape(int M, int B) {
  if (B <= 16) return {};
  const long long bt = (B + 15) / 16;  // batch tiles of 16 rows
  struct Cand {
    int rt, nbt;
  };
  constexpr Cand kCands[] = {{1, 2}, {2, 2}, {4, 2}, {4, 4}};
  Cand pick{0, 0}, prev{0, 0};
  long long w_pick = 0, w_prev = 0;
  for (const Cand& c : kCands) {
    if (c.nbt == 4 && bt < 3) continue;
    const long long w = (long long)((M + 16 * c.rt - 1) / (16 * c.rt)) * ((bt + c.nbt - 1) / c.nbt);
    if (w <= 256) {
      if (w >= 144) {
        pick = c;
        w_pick = w;
      } else if (prev.rt) {
        pick = prev;
        w_pick = w_prev;
      }
      break;
    }
    prev = c;
    w_prev = w;
  }
  if (!pick.rt && w_prev > 256) {  // no shape fits one round: the most reuse
    pick = prev;
    w_pick = w_prev;
  }
  if (!pick.rt || (pick.rt == 1 && B <= 32)) return {};
  const bool two_per_cu = pick.rt == 4 && pick.nbt == 4 && w_pick > 256 && w_pick <= 512;
  return {two_per_cu ? 2 : 4, pick.rt, pick.nbt};
}

// A shape of the double-buffered tiles (gemv_reuse_pf): KS waves, RT tiles
// per wave, XL x loads per block; KS = 0: not these tiles.
struct PfShape {
  int ks = 0, rt = 0, xl = 0;
};

// Where the double-buffered tiles take the single pass (paired scales
// only). From a sweep of every tile kernel, timed back to back over cold
// weights, us,
// the double-buffered tiles against the best single-buffered ones in
// brackets; from 9 batch rows 4 waves with 8 x loads per block:
//                        B = 12         B = 16         B = 32
//   M = K = 4096:        4.88 (5.17)    4.97 (5.45)    6.50 (6.37)
//   M = 4096, K = 11008: 9.44 (9.59)    10.00 (10.76)  12.94 (13.39)
//   M = 3072, K = 8192:  7.36 (7.81)    7.76 (8.52)    10.02 (10.58)
//   M = 2048, K = 16384: 11.53 (12.01)  12.33 (13.62)  12.24 (13.44)
//   M = 2048, K = 4096:  4.73 (4.87)    4.79 (5.09)    4.79 (5.13)
//   M = 6144, K = 8192:  10.44 (10.73)  10.82 (11.46)  19.33 (18.67)
//   M = 8192, K = 28672: 29.74 (31.51)  33.20 (34.60)  66.16 (63.84)
//   M = 5120, K = 5120:  8.07 (7.48)    8.16 (7.92)    14.11 (11.76)
//   M = 28672, K = 8192: 36.79 (37.13)  39.34 (38.62)  70.05 (66.75)
// Up to 8 batch rows (one batch tile) 4 or 2 x loads per block (XL), the x
// buffers holding only those 8 or 4 rows (the MFMA reads zeros for the
// rest), which leaves room for two workgroups per CU:
//                        B = 3               B = 5               B = 8
//   M = K = 4096:        4.34 (4.41) 6,1,2   4.37 (4.60) 6,1,4   4.56 (4.87) 6,1,4
//   M = 3072, K = 8192:  6.01 (6.20) 8,1,4   6.22 (6.77) 8,1,4   6.61 (7.01) 8,1,4
//   M = 2048, K = 16384: (stream 7.86)       9.15 (9.73) 8,1,4   9.83 (10.73) 8,1,4
//   M = 11008, K = 4096: 7.50 (7.65) 4,1,2   7.82 (7.96) 4,1,4   8.32 (9.13) 4,1,4
//   M = 28672, K = 8192: 25.42 (27.56) 4,1,2 27.53 (28.85) 4,2,4 29.45 (33.47) 4,2,4
//   M = 6144, K = 8192:  8.96 (8.92) 4,2,4   9.03 (9.10) 4,2,4   9.24 (9.88) 4,2,4
// (KS, RT, XL after each). The single-buffered tiles keep 3-5 batch rows on
// rows longer than 8192 weights at 2049-4096 rows (M = 4096, K = 11008,
// B = 4: 7.32 against 7.62) and rows shorter than 8192 at 4097-8192 rows up
// to 5 (M = 5120, K = 5120, B = 3: 6.21 against 6.54), above 16 batch rows
// at 4097+ rows and from 9 above 8192 rows, and at M <= 1024 above 32
// batch rows (three batch tiles) on rows shorter than 16384 weights
// (M = 512, K = 8192, B = 33: 6.40 against 6.71).
// Above 8192 rows, two tiles per wave from 12289 rows, one below (an
// earlier rule, the one the table above was timed with, took two tiles on
// rows longer than 4096 weights and one otherwise; us, against it in
// brackets):
//   M = 9216, K = 8192, B = 5: 13.54 (14.84)   M = 11008, K = 8192, B = 5: 13.87 (15.01)
//   M = 12288, K = 8192, B = 8: 15.53 (16.23)  M = 14336, K = 4096, B = 8: 9.45 (10.29)
//   M = 16384, K = 4096, B = 8: 9.60 (10.65)   M = 28672, K = 4096, B = 8: 15.59 (16.78)
//   M = 14336, K = 8192, B = 4: 14.74 (16.04)  M = 28672, K = 8192, B = 4: 25.90 (26.69)
// (M = 28672 and 14336 at K = 8192, B = 5-8 keep two tiles.)
PfShape reuse_pf_shape(int M, int K, int B) {
  if (M > 8192) {
    if (B > 8) return {};
    const int rt = M > 12288 ? 2 : 1;
    return {4, rt, B <= 4 ? 2 : 4};
  }
  if (M > 4096) {
    if (B >= 9 && B <= 16 && K >= 8192) return {4, 2, 8};
    if (B <= 8 && (K >= 8192 || B >= 6)) return {4, 2, 4};
    return {};
  }
  if (M > 2048) {
    if (B > 16) return K >= 8192 ? PfShape{4, 2, 8} : PfShape{};
    if (B >= 9) return {4, 1, 8};
    if (K <= 4096) return B <= 4 ? PfShape{6, 1, 2} : PfShape{6, 1, 4};
    if (K > 8192 && B <= 5) return {};
    return {8, 1, 4};
  }
  if (B >= 9) return M <= 1024 && B > 32 && K < 16384 ? PfShape{} : PfShape{4, 1, 8};
  if (B < 5) return {};
  return K >= 8192 ? PfShape{8, 1, 4} : PfShape{6, 1, 4};
}

// The single-pass tiles. Where the double-buffered tiles do not run
// (reuse_pf_shape, or scales that do not pair), the single-buffered LDS-staged
// kernel (gemv_reuse_lds) against the tiles that load the MFMA operands
// directly (gemv_reuse) in brackets, us per launch, from an earlier sweep:
//                        B = 4          B = 8          B = 16         B = 32
//   M = K = 4096:        4.65 (4.62)    4.94 (5.01)    5.58 (6.78)    6.37 (7.82)
//   M = 4096, K = 11008: 7.84 (8.40)    8.85 (10.65)   10.97 (15.20)  13.24 (16.92)
//   M = 3072, K = 8192:  6.60 (6.74)    7.36 (7.69)    8.56 (11.30)   10.58 (13.17)
//   M = 2048, K = 8192:                 7.12 (7.52)    8.25 (11.09)   8.08 (11.08)
//   M = 5120, K = 5120:  6.43 (6.55)    7.04 (7.75)    7.83 (10.03)   11.76 (16.51)
//   M = 6144, K = 8192:  9.20 (9.15)    10.10 (11.14)  11.58 (14.69)  18.98 (23.78)
//   M = 8192, K = 28672: 25.70 (26.18)  29.02 (32.87)  34.79 (41.08)  64.65 (77.98)
//   M = 11008, K = 4096: 8.42 (8.84)    9.42 (10.12)   11.21 (13.05)  15.25 (18.63)
//   M = 28672, K = 8192: 30.64 (28.43)  34.18 (34.22)  39.05 (44.75)  66.82 (77.26)
// Up to 4096 rows (256 tiles) one tile per wave: 16 waves, or 8 at 6-8
// batch rows of up to 8192 weights (M = 3072, K = 8192, B = 8: 7.05
// against 7.31) while 16 keep up to 5 (B = 3: 6.25 against 6.86); two per
// wave above 16 batch rows (the grid then has two batch tiles); to 8192
// rows two tiles per wave, 8 waves (4 above 16 batch rows: M = 6144,
// K = 8192, B = 32 18.98 against 20.24); above, 4 waves (two tiles per wave
// from 9 batch rows). The direct tiles stay at M = 28672, K = 8192 up to 8
// batch rows (B = 3: 27.79 against 29.80) and on rows of up to 4096 weights
// at 2049-4096 rows up to 5 batch rows (M = K = 4096: B = 3 4.53 against
// 4.60, B = 5 4.61 against 4.77).
int launch_reuse_tiles(const Launch& L, const uint4* p, const uint16_t* s, const uint4* x,
                       uint16_t* y, int M, int K, int B) {
  if ((K / DK_GROUP_SIZE) % 2 == 0 && aligned(s, 4)) {
    const PfbShape pfb = reuse_pfb_shape(M, B);
    if (pfb.rt == 4 && pfb.nbt == 4)
      return pfb.ks == 2 ? launch_reuse_pfb<2, 4, 4>(L, p, s, x, y, M, K, B)
                         : launch_reuse_pfb<4, 4, 4>(L, p, s, x, y, M, K, B);
    if (pfb.rt == 4) return launch_reuse_pfb<4, 4, 2>(L, p, s, x, y, M, K, B);
    if (pfb.rt == 2) return launch_reuse_pfb<4, 2, 2>(L, p, s, x, y, M, K, B);
    if (pfb.rt == 1) return launch_reuse_pfb<4, 1, 2>(L, p, s, x, y, M, K, B);
    const PfShape pf = reuse_pf_shape(M, K, B);
    if (pf.ks == 8) return launch_reuse_pf<8, 1, 4>(L, p, s, x, y, M, K, B);
    if (pf.ks == 6)
      return pf.xl == 2 ? launch_reuse_pf<6, 1, 2>(L, p, s, x, y, M, K, B)
                        : launch_reuse_pf<6, 1, 4>(L, p, s, x, y, M, K, B);
    if (pf.ks == 4 && pf.rt == 1) {
      if (pf.xl == 2) return launch_reuse_pf<4, 1, 2>(L, p, s, x, y, M, K, B);
      if (pf.xl == 4) return launch_reuse_pf<4, 1, 4>(L, p, s, x, y, M, K, B);
      return launch_reuse_pf<4, 1, 8>(L, p, s, x, y, M, K, B);
    }
    if (pf.ks == 4 && pf.rt == 2) {
      if (pf.xl == 2) return launch_reuse_pf<4, 2, 2>(L, p, s, x, y, M, K, B);
      return pf.xl == 8 ? launch_reuse_pf<4, 2, 8>(L, p, s, x, y, M, K, B)
                        : launch_reuse_pf<4, 2, 4>(L, p, s, x, y, M, K, B);
    }
  }
  if (M > 2048 && M <= 4096 && K <= 4096 && B <= 5)
    return launch_reuse<8, 1, 2>(L, p, s, x, y, M, K, B);
  if (M > 8192) {
    if (B <= 8 && K > 4096) return launch_reuse<8, 2, 2>(L, p, s, x, y, M, K, B);
    return B <= 8 ? launch_reuse_lds<4, 1>(L, p, s, x, y, M, K, B)
                  : launch_reuse_lds<4, 2>(L, p, s, x, y, M, K, B);
  }
  if (M > 4096)
    return B <= 16 ? launch_reuse_lds<8, 2>(L, p, s, x, y, M, K, B)
                   : launch_reuse_lds<4, 2>(L, p, s, x, y, M, K, B);
  if (M > 2048 && B > 16) return launch_reuse_lds<8, 2>(L, p, s, x, y, M, K, B);
  if (M > 2048 && B >= 6 && B <= 8 && K <= 8192) return launch_reuse_lds<8, 1>(L, p, s, x, y, M, K, B);
  // Up to 2048 rows of 8192 weights or more, from 9 batch rows: blocks of
  // four groups, 8 waves (one block per wave at K = 8192; us, against 16
  // waves with blocks of two): M = 2048, K = 16384, B = 16 12.92 (13.81),
  // B = 32 12.91 (13.45); M = 2048, K = 8192, B = 16 8.04 (8.34). At 8
  // batch rows, and above 32 at M <= 1024, blocks of two with 8 waves
  // (against blocks of four): M = 2048, K = 8192, B = 8 6.76 (7.06);
  // M = 1024, K = 8192, B = 33 6.63 (7.39). At M = K = 4096 blocks of four
  // lose (B = 16: 5.83 against 5.61).
  if (M <= 2048 && K >= 8192 && B >= 8) {
    if (B == 8 || (M <= 1024 && B > 32)) return launch_reuse_lds<8, 1>(L, p, s, x, y, M, K, B);
    return launch_reuse_lds<8, 1, 4>(L, p, s, x, y, M, K, B);
  }
  return launch_reuse_lds<16, 1>(L, p, s, x, y, M, K, B);
}

// h of the MLP step at the start of its workspace, padded to 256 bytes so
// that the down projection's split-K workspace after it stays aligned.
size_t mlp_h_bytes(int I, int B) { return ((size_t)B * (size_t)I * sizeof(uint16_t) + 255) / 256 * 256; }

// Split-K tiles: S workgroups per tile, the tickets (8 bytes per tile and
// batch tile) first in the workspace, then the fp32 partials [S][B][M].
size_t split_tickets(int M, int B) {
  return (size_t)((M + 15) / 16) * (size_t)((B + dk::kReuseBatch - 1) / dk::kReuseBatch);
}

size_t split_ticket_bytes(int M, int B) { return (split_tickets(M, B) * 8 + 255) / 256 * 256; }

int reuse_split_slices(int M, int K, int B);

size_t split_workspace_bytes(int M, int K, int B) {
  return split_ticket_bytes(M, B) + (size_t)reuse_split_slices(M, K, B) * B * M * sizeof(float);
}

// Generation of a split call (take_ticket): distinct for every launch in a
// process, 58 bits shifted above the 6-bit arrival count.
std::atomic<unsigned long long> g_ticket_gen{0x2545F4914F6CDD1Dull};

unsigned long long next_gen() {
  return (g_ticket_gen.fetch_add(1ull, std::memory_order_relaxed) & ((1ull << 58) - 1ull)) << 6;
}

// The double-buffered split tiles (4 waves, one tile each) where the scales
// come in pairs; else the tiles that load the MFMA operands directly, two
// per wave of 8 (their tickets, one per pair of tiles, fit the same
// workspace).
int launch_reuse_split(const Launch& L, const uint4* p, const uint16_t* s, const uint4* x,
                       uint16_t* y, int M, int K, int B, void* workspace) {
  const int S = reuse_split_slices(M, K, B);
  auto* tickets = static_cast<unsigned long long*>(workspace);
  auto* partials =
      reinterpret_cast<float*>(static_cast<char*>(workspace) + split_ticket_bytes(M, B));
  const int bt = (B + dk::kReuseBatch - 1) / dk::kReuseBatch;
  if ((K / DK_GROUP_SIZE) % 2 == 0 && aligned(s, 4))
    return L("reuse split launch", dk::gemv_reuse_split_pf<4, 1>, dim3((M + 15) / 16, bt, S),
             dim3(4 * 64), 0, p, s, x, y, partials, tickets, next_gen(), M, K, B);
  return L("reuse split launch", dk::gemv_reuse_split<8, 2, 2>, dim3((M + 31) / 32, bt, S),
           dim3(8 * 64), 0, p, s, x, y, partials, tickets, next_gen(), M, K, B);
}

enum class ReuseShape { kStream, kTiles };

// Which kernel the reuse path takes, from a sweep of the tile kernels (both
// forms, 4-16 waves, one or two tiles per wave) against the streaming
// kernel at 3-32 batch rows on 11 shapes, timed back to back over cold
// weights, us:
//   M = 2048, K = 16384: B = 4 stream 9.02 (tiles 9.37), B = 5 tiles 9.97 (stream 10.80)
//   M = 2048, K = 8192:  B = 4 stream 5.74 (6.19), B = 8 tiles 7.12 (7.66)
//   M = 1024, K = 4096:  B = 8 stream 3.73 (4.64), B = 12 tiles 4.87 (4.99)
//   M = 4096, K = 11008, B = 3: tiles 7.50 (stream 9.63)
//   M = 3072, K = 8192,  B = 3: tiles 6.40 (stream 7.11)
//   M = 6144, K = 8192,  B = 3: tiles 9.14 (stream 10.45)
//   M = 11008, K = 4096, B = 3: tiles 7.82 (stream 8.51)
//   M = 8192, K = 3584,  B = 3: tiles 5.77 (stream 6.43)
//   M = 2560, K = 8192,  B = 4: tiles 6.27 (stream 9.61)
//   M = K = 4096,        B = 3: tiles 4.33 (stream 4.54; double buffered)
//   M = 2048, K = 4096,  B = 8: tiles 4.30 (stream 4.71; double buffered)
// Up to 512 rows the streaming kernel keeps every batch up to 32 rows (M =
// 512, K = 8320, B = 32: 11.67 against 11.47 for the earlier tiles); it also
// keeps up to four batch rows at M <= 2048, and up to eight there on rows
// shorter than 8192 weights with an odd number of groups (the
// double-buffered tiles need pairs of groups; the single-buffered ones
// were level with the streaming kernel: M = 2048, K = 4096, B = 8 4.65
// against 4.68).
// Where the groups pair (`pairs`: an even group count and 4-byte aligned
// scales), the double-buffered tiles also take two batch rows above 12288
// rows and three at 4097-8191 rows on rows of up to 4096 weights, found by
// timing them at shapes the streaming kernel kept (us, streaming in
// brackets): B = 2, M = 14336, K = 8192 14.30 (15.63); M = 16384, K = 4096
// 8.45 (9.75); M = 13824, K = 5120 9.94 (11.83); M = 28672, K = 8192 25.00
// (25.80); B = 3 at K = 2048 / 3072 / 4096, M = 6144: 4.14 / 4.90 / 5.62
// (5.95 / 6.12 / 6.21), M = 4608 and 7168 alike.
ReuseShape reuse_shape(int M, int K, int B, bool pairs) {
  if (B == 2 && pairs && M > 12288) return ReuseShape::kTiles;
  if (B <= 2 || M <= 128) return ReuseShape::kStream;
  if (M <= 512) return B <= 32 ? ReuseShape::kStream : ReuseShape::kTiles;
  if (M <= 1024) return B < 12 ? ReuseShape::kStream : ReuseShape::kTiles;
  if (M <= 2048 && (B <= 4 || (B <= 8 && K < 8192 && (K / DK_GROUP_SIZE) % 2 == 1)))
    return ReuseShape::kStream;
  if (B == 3) {
    const bool tiles = K >= 8192 || M >= 8192 || (size_t)M * (size_t)K >= ((size_t)1 << 27) ||
                       (M >= 3072 && K > 4096 && K < 8192) || (M > 2048 && M <= 4096 && K <= 4096) ||
                       (pairs && M > 4096 && K <= 4096);
    return tiles ? ReuseShape::kTiles : ReuseShape::kStream;
  }
  return ReuseShape::kTiles;
}

// The tiles split K over S workgroups per tile, given a workspace, where a
// tile per workgroup leaves most CUs idle and the rows are long: up to 64
// tiles (M <= 1024 at 16 batch rows) on rows of 16384+ weights, up to 128
// on rows of 28672+. The reduction across workgroups costs several
// microseconds on this 8-XCD part (the partials and tickets pass the
// non-coherent L2s), so the rows must be long enough to repay it. From the
// sweep of the double-buffered tiles (us; single-pass tiles, then the
// earlier split of 8 waves with two tiles each, in brackets):
//   M = 1024, K = 16384, B = 16: S = 2 11.61 (12.11, 15.75)
//   M = 1024, K = 28672, B = 16: S = 4 14.63 (20.97, 20.36)
//   M = 512,  K = 28672, B = 33: S = 2 14.74 (17.87, 20.60)
//   M = 600,  K = 65536, B = 16: S = 4 19.44 (40.85, 32.77)
// and single-pass where it lost: M = 1024, K = 28672, B = 33: 18.27 (S = 2
// 24.18); M = 1024, K = 14336, B = 16: 11.44 (S = 2 11.32, S = 4 12.13).
int reuse_split_slices(int M, int K, int B) {
  if (reuse_shape(M, K, B, false) != ReuseShape::kTiles || M > 1024) return 0;
  const long long tiles = (long long)((M + 15) / 16) * ((B + dk::kReuseBatch - 1) / dk::kReuseBatch);
  if (tiles <= 64 && K >= 28672) return 4;
  if (tiles <= 64 && K >= 16384) return 2;
  if (tiles <= 128 && K >= 28672) return 2;
  return 0;
}

bool reuse_split(int M, int K, int B) { return reuse_split_slices(M, K, B) > 0; }

size_t v3_lds_bytes(int K) { return (size_t)kWavesPerBlock * (K / DK_GROUP_SIZE) * sizeof(uint16_t); }

int check_io(const uint32_t* packed, const uint16_t* scales, const uint16_t* x, const uint16_t* y) {
  if (!packed || !scales || !x || !y)
    return fail(DK_ERR_INVALID_ARGUMENT, "packed, scales, x and y must not be NULL");
  if (!aligned(packed, 16) || !aligned(x, 16))
    return fail(DK_ERR_INVALID_ARGUMENT, "packed and x must be 16-byte aligned");
  if (!aligned(scales, 2) || !aligned(y, 2))
    return fail(DK_ERR_INVALID_ARGUMENT, "scales and y must be 2-byte aligned");
  return DK_OK;
}

int gemv_impl(const uint32_t* packed, const uint16_t* scales, const uint16_t* x, uint16_t* y, int M,
              int K, int B, const dk_gemv_config* cfg, void* workspace, size_t workspace_bytes,
              const Launch& L) {
  int rc = dk_gemv_validate(M, K, B, cfg);
  if (rc != DK_OK) return rc;
  if (M <= 0 || K <= 0 || B <= 0) return DK_OK;
  rc = check_io(packed, scales, x, y);
  if (rc != DK_OK) return rc;
  const size_t need = dk_gemv_workspace_bytes(M, K, B, cfg);
  // The reuse path's split-K tiles run when a large enough workspace comes
  // with the call; without one it runs the single-pass tiles.
  const bool split = cfg->reuse_weights && need > 0 && workspace && workspace_bytes >= need;
  if (need > 0 && !cfg->reuse_weights) {
    if (!workspace || workspace_bytes < need)
      return fail(DK_ERR_INVALID_ARGUMENT, "split-K needs a %zu-byte workspace (got %zu)", need,
                  workspace_bytes);
    if (!aligned(workspace, 8)) return fail(DK_ERR_INVALID_ARGUMENT, "workspace must be 8-byte aligned");
  }
  if (split && !aligned(workspace, 8))
    return fail(DK_ERR_INVALID_ARGUMENT, "workspace must be 8-byte aligned");

  const uint4* p4 = reinterpret_cast<const uint4*>(packed);
  const uint4* x4 = reinterpret_cast<const uint4*>(x);

  if (cfg->reuse_weights) {
    const bool pairs = (K / DK_GROUP_SIZE) % 2 == 0 && aligned(scales, 4);
    if (reuse_shape(M, K, B, pairs) == ReuseShape::kStream)
      return L.stamp(launch_v5<dk::LayoutLogical, DK_STAMP_REUSE>(L, p4, scales, x4, y, M, K, B),
                     DK_STAMP_REUSE);
    if (split)
      return L.stamp(launch_reuse_split(L, p4, scales, x4, y, M, K, B, workspace), DK_STAMP_REUSE);
    return L.stamp(launch_reuse_tiles(L, p4, scales, x4, y, M, K, B), DK_STAMP_REUSE);
  }
  const dim3 block4(kWavesPerBlock * 64);
  const dim3 rows4((M + kWavesPerBlock - 1) / kWavesPerBlock);
  switch (cfg->version) {
    case DK_V0:
      return L.stamp(L("v0 launch", dk::gemv_v0, dim3((M + 255) / 256), dim3(256), 0, packed,
                       scales, x, y, M, K, B),
                     DK_V0);
    case DK_V1:
      if (cfg->warps_per_row > 1) {
        const int wpr = clamp_wpr(cfg->warps_per_row);
        return L.stamp(L("v1 multiwave launch", dk::gemv_v1_multiwave, dim3(M), dim3(wpr * 64), 0,
                         packed, scales, x4, y, M, K, B),
                       DK_STAMP_MULTIWAVE_BASE + wpr);
      }
      return L.stamp(L("v1 launch", dk::gemv_v1, rows4, block4, 0, packed, scales, x4, y, M, K, B),
                     DK_V1);
    case DK_V2:
      return L.stamp(
          L("v2 launch", dk::gemv_v23<false>, rows4, block4, 0, p4, scales, x4, y, M, K, B), DK_V2);
    case DK_V3:
      return L.stamp(L("v3 launch", dk::gemv_v23<true>, rows4, block4, v3_lds_bytes(K), p4, scales,
                       x4, y, M, K, B),
                     DK_V3);
    case DK_V4:
      return L.stamp(launch_v4(L, p4, scales, x4, y, nullptr, M, K, B, cfg->split_k), DK_V4);
    case DK_V5:
      return L.stamp(launch_v5(L, p4, scales, x4, y, M, K, B), DK_V5);
    default:
      return fail(DK_ERR_INVALID_ARGUMENT, "unknown version %d", cfg->version);
  }
}

// The reference's workspace contract: v4 leaves the fp32 sums in the
// caller's [B, M] buffer `acc` (the reference accumulated them there and
// converted them to y); every other variant runs as dk_w4a16_gemv without a
// workspace.
int gemv_ref_workspace_impl(const uint32_t* packed, const uint16_t* scales, const uint16_t* x,
                            uint16_t* y, int M, int K, int B, const dk_gemv_config* cfg,
                            float* acc, const Launch& L) {
  int rc = dk_gemv_validate(M, K, B, cfg);
  if (rc != DK_OK) return rc;
  if (cfg->reuse_weights || cfg->version != DK_V4)
    return gemv_impl(packed, scales, x, y, M, K, B, cfg, nullptr, 0, L);
  if (M <= 0 || K <= 0 || B <= 0) return DK_OK;
  rc = check_io(packed, scales, x, y);
  if (rc != DK_OK) return rc;
  if (!acc)
    return fail(DK_ERR_INVALID_ARGUMENT, "v4 needs the caller-zeroed fp32 [B, M] workspace");
  if (!aligned(acc, 4)) return fail(DK_ERR_INVALID_ARGUMENT, "workspace must be 4-byte aligned");
  return L.stamp(launch_v4(L, reinterpret_cast<const uint4*>(packed), scales,
                           reinterpret_cast<const uint4*>(x), y, acc, M, K, B, cfg->split_k),
                 DK_V4);
}

}  // namespace

// ---------------------------------------------------------------------------
// Library-owned scratch for dk_w4a16_gemv_noalloc: the workspace of the
// reuse path's split-K tiles in a file-scope device array, so that a call
// allocates nothing. Every GPU the library runs
// on holds its own copy (DK_NOALLOC_SCRATCH_BYTES) until the process ends. Its
// device address is taken once per device with hipGetSymbolAddress, with
// that device current, and only that address is used from the host (the
// array's name is a host-side stand-in). Nothing in it must start at zero:
// the tickets carry each call's generation (take_ticket), and the partials
// are written before they are read. Calls that overlap in time on one GPU
// share it and race.
// ---------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[DK_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr size_t kNoallocScratchBytes = DK_NOALLOC_SCRATCH_BYTES;

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// The current device's address of `scratch` (set up on the first call on
// that device).
int scratch_ptr(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return dk::hip_error(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices)
    return fail(DK_ERR_UNSUPPORTED, "device %d beyond the %d devices the scratch supports", dev,
                kMaxDevices);
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return dk::hip_error(e, "hipGetSymbolAddress(scratch)");
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return DK_OK;
}

}  // namespace

extern "C" {

void dk_gemv_config_default(dk_gemv_config* cfg) {
  if (!cfg) return;
  cfg->version = DK_V5;
  cfg->split_k = 4;
  cfg->reuse_weights = 0;
  cfg->warps_per_row = 1;
}

int dk_gemv_validate(int M, int K, int B, const dk_gemv_config* cfg) {
  if (!cfg) return fail(DK_ERR_INVALID_ARGUMENT, "cfg must not be NULL");
  if (cfg->version < 0 || cfg->version > 5) return fail(DK_ERR_INVALID_ARGUMENT, "version must be 0..5");
  if (cfg->split_k < 1 || cfg->split_k > 32)
    return fail(DK_ERR_INVALID_ARGUMENT, "split_k must be in [1, 32]");
  if (cfg->warps_per_row < 1 || cfg->warps_per_row > 8)
    return fail(DK_ERR_INVALID_ARGUMENT, "warps_per_row must be in [1, 8]");
  if (cfg->warps_per_row > 1 && (cfg->version != DK_V1 || cfg->reuse_weights))
    return fail(DK_ERR_INVALID_ARGUMENT, "warps_per_row > 1 is implemented for streaming v1 only");
  if (M <= 0 || K <= 0 || B <= 0) return DK_OK;  // no-op call
  if (K % DK_GROUP_SIZE != 0) return fail(DK_ERR_INVALID_ARGUMENT, "K must be divisible by group size 128");
  if (K > (1 << 28)) return fail(DK_ERR_UNSUPPORTED, "K=%d exceeds the supported 2^28", K);
  // v5 addresses activations through one buffer descriptor with 32-bit offsets.
  if ((long long)B * K * 2 > 0x7fffffffLL)
    return fail(DK_ERR_UNSUPPORTED, "B*K=%lld activation elements exceed 2^30", (long long)B * K);
  if (!cfg->reuse_weights && cfg->version == DK_V3) {
    if (v3_lds_bytes(K) > (size_t)lds_limit_bytes())
      return fail(DK_ERR_UNSUPPORTED, "K=%d needs %zu B of LDS on v3 (limit %d)", K, v3_lds_bytes(K),
                  lds_limit_bytes());
  }
  return DK_OK;
}

size_t dk_gemv_workspace_bytes(int M, int K, int B, const dk_gemv_config* cfg) {
  if (dk_gemv_validate(M, K, B, cfg) != DK_OK) return 0;
  if (M <= 0 || K <= 0 || B <= 0) return 0;
  if (cfg->reuse_weights) return reuse_split(M, K, B) ? split_workspace_bytes(M, K, B) : 0;
  return 0;
}

int dk_w4a16_gemv(const uint32_t* packed, const uint16_t* scales, const uint16_t* x, uint16_t* y,
                  int M, int K, int B, const dk_gemv_config* cfg, void* workspace,
                  size_t workspace_bytes, hipStream_t stream) {
  return gemv_impl(packed, scales, x, y, M, K, B, cfg, workspace, workspace_bytes, Launch{stream});
}

int dk_w4a16_gemv_noalloc(const uint32_t* packed, const uint16_t* scales, const uint16_t* x,
                          uint16_t* y, int M, int K, int B, const dk_gemv_config* cfg,
                          hipStream_t stream) {
  int rc = dk_gemv_validate(M, K, B, cfg);
  if (rc != DK_OK) return rc;
  if (M <= 0 || K <= 0 || B <= 0) return DK_OK;
  const size_t need = dk_gemv_workspace_bytes(M, K, B, cfg);
  if (need == 0) return gemv_impl(packed, scales, x, y, M, K, B, cfg, nullptr, 0, Launch{stream});
  if (need > kNoallocScratchBytes)
    return fail(DK_ERR_UNSUPPORTED,
                "split-K needs %zu bytes of workspace; dk_w4a16_gemv_noalloc holds %zu (call "
                "dk_w4a16_gemv, with or without a workspace)",
                need, kNoallocScratchBytes);
  rc = check_io(packed, scales, x, y);
  if (rc != DK_OK) return rc;
  void* ws = nullptr;
  rc = scratch_ptr(&ws);
  if (rc != DK_OK) return rc;
  return gemv_impl(packed, scales, x, y, M, K, B, cfg, ws, kNoallocScratchBytes, Launch{stream});
}

int dk_w4a16_gemv_ref_workspace(const uint32_t* packed, const uint16_t* scales, const uint16_t* x,
                                uint16_t* y, int M, int K, int B, const dk_gemv_config* cfg,
                                float* workspace, hipStream_t stream) {
  return gemv_ref_workspace_impl(packed, scales, x, y, M, K, B, cfg, workspace, Launch{stream});
}

int dk_gemv_describe(int M, int K, int B, const dk_gemv_config* cfg, size_t workspace_bytes,
                     dk_launch_info* info) {
  if (!info) return fail(DK_ERR_INVALID_ARGUMENT, "info must not be NULL");
  *info = dk_launch_info{};
  // Placeholder addresses with every alignment the checks ask for; in
  // describe mode nothing is launched and nothing is dereferenced.
  const auto* p = reinterpret_cast<const uint32_t*>(uintptr_t{4096});
  const auto* h = reinterpret_cast<const uint16_t*>(uintptr_t{4096});
  void* ws = workspace_bytes > 0 ? reinterpret_cast<void*>(uintptr_t{4096}) : nullptr;
  Launch L{nullptr, info};
  return gemv_impl(p, h, h, const_cast<uint16_t*>(h), M, K, B, cfg, ws, workspace_bytes, L);
}

int dk_last_kernel_stamp(void) {
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    dk::hip_error(e, "hipDeviceSynchronize");
    return -1;
  }
  int dev = 0;
  e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    dk::hip_error(e, "hipGetDevice");
    return -1;
  }
  if (dev < 0 || dev >= kStampDevices) return -1;
  return g_stamps[dev].exchange(0, std::memory_order_relaxed) - 1;
}

int dk_w4a16_gemv_paired(const uint32_t* paired, const uint16_t* scales, const uint16_t* x,
                         uint16_t* y, int M, int K, int B, hipStream_t stream) {
  dk_gemv_config cfg;
  dk_gemv_config_default(&cfg);
  int rc = dk_gemv_validate(M, K, B, &cfg);
  if (rc != DK_OK) return rc;
  if (M <= 0 || K <= 0 || B <= 0) return DK_OK;
  if (!paired || !scales || !x || !y)
    return fail(DK_ERR_INVALID_ARGUMENT, "paired, scales, x and y must not be NULL");
  if (!aligned(paired, 16) || !aligned(x, 16))
    return fail(DK_ERR_INVALID_ARGUMENT, "paired and x must be 16-byte aligned");
  if (!aligned(scales, 2) || !aligned(y, 2))
    return fail(DK_ERR_INVALID_ARGUMENT, "scales and y must be 2-byte aligned");
  const Launch L{stream};
  return L.stamp(launch_v5<dk::LayoutPaired>(L, reinterpret_cast<const uint4*>(paired), scales,
                                             reinterpret_cast<const uint4*>(x), y, M, K, B),
                 DK_STAMP_PAIRED);
}

int dk_gate_up_silu(const uint32_t* gate_packed, const uint16_t* gate_scales,
                    const uint32_t* up_packed, const uint16_t* up_scales, const uint16_t* x,
                    uint16_t* h, int I, int H, int B, hipStream_t stream) {
  if (I <= 0 || H <= 0 || B <= 0) return DK_OK;
  if (H % DK_GROUP_SIZE != 0)
    return fail(DK_ERR_INVALID_ARGUMENT, "H=%d must be divisible by group size 128", H);
  if (H > (1 << 28)) return fail(DK_ERR_UNSUPPORTED, "H=%d exceeds the supported 2^28", H);
  if ((long long)B * H * 2 > 0x7fffffffLL)
    return fail(DK_ERR_UNSUPPORTED, "B*H=%lld activation elements exceed 2^30", (long long)B * H);
  if (!gate_packed || !gate_scales || !up_packed || !up_scales || !x || !h)
    return fail(DK_ERR_INVALID_ARGUMENT, "gate, up, their scales, x and h must not be NULL");
  if (!aligned(gate_packed, 16) || !aligned(up_packed, 16) || !aligned(x, 16))
    return fail(DK_ERR_INVALID_ARGUMENT, "gate, up and x must be 16-byte aligned");
  if (!aligned(gate_scales, 2) || !aligned(up_scales, 2) || !aligned(h, 2))
    return fail(DK_ERR_INVALID_ARGUMENT, "scales and h must be 2-byte aligned");
  const Launch L{stream};
  return L.stamp(launch_gate_up(L, reinterpret_cast<const uint4*>(gate_packed), gate_scales,
                                reinterpret_cast<const uint4*>(up_packed), up_scales,
                                reinterpret_cast<const uint4*>(x), h, I, H, B),
                 DK_STAMP_GATE_UP);
}

size_t dk_mlp_workspace_bytes(int I, int H, int B) {
  if (I <= 0 || H <= 0 || B <= 0) return 0;
  dk_gemv_config cfg;
  dk_gemv_config_default(&cfg);
  cfg.reuse_weights = B > 1 ? 1 : 0;
  return mlp_h_bytes(I, B) + dk_gemv_workspace_bytes(H, I, B, &cfg);
}

int dk_mlp_decode(const uint32_t* gate_packed, const uint16_t* gate_scales,
                  const uint32_t* up_packed, const uint16_t* up_scales,
                  const uint32_t* down_packed, const uint16_t* down_scales, const uint16_t* x,
                  uint16_t* y, int I, int H, int B, void* workspace, size_t workspace_bytes,
                  hipStream_t stream) {
  if (I <= 0 || H <= 0 || B <= 0) return DK_OK;
  if (I % DK_GROUP_SIZE != 0)
    return fail(DK_ERR_INVALID_ARGUMENT, "I=%d must be divisible by group size 128", I);
  // h is required; the down projection's split-K workspace after it is used
  // when the caller provides dk_mlp_workspace_bytes() in full.
  const size_t need_h = (size_t)B * (size_t)I * sizeof(uint16_t);
  if (!workspace || workspace_bytes < need_h)
    return fail(DK_ERR_INVALID_ARGUMENT, "the MLP step needs a %zu-byte workspace (got %zu)",
                need_h, workspace_bytes);
  if (!aligned(workspace, 16)) return fail(DK_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
  dk_gemv_config cfg;
  dk_gemv_config_default(&cfg);
  // The down projection takes the weight-reuse path for a batch, as
  // w4a16_linear does (python/decode_kernel/__init__.py:71-74): the v5
  // kernel up to a few rows, the MFMA tiles beyond.
  cfg.reuse_weights = B > 1 ? 1 : 0;
  // Validate the down projection before anything is launched.
  int rc = dk_gemv_validate(H, I, B, &cfg);
  if (rc != DK_OK) return rc;
  if (!down_packed || !down_scales || !y)
    return fail(DK_ERR_INVALID_ARGUMENT, "down, its scales and y must not be NULL");
  if (!aligned(down_packed, 16)) return fail(DK_ERR_INVALID_ARGUMENT, "down must be 16-byte aligned");
  if (!aligned(down_scales, 2) || !aligned(y, 2))
    return fail(DK_ERR_INVALID_ARGUMENT, "scales and y must be 2-byte aligned");
  uint16_t* h = static_cast<uint16_t*>(workspace);
  rc = dk_gate_up_silu(gate_packed, gate_scales, up_packed, up_scales, x, h, I, H, B, stream);
  if (rc != DK_OK) return rc;
  const size_t down_ws = dk_gemv_workspace_bytes(H, I, B, &cfg);
  const bool with_split = down_ws > 0 && workspace_bytes >= mlp_h_bytes(I, B) + down_ws;
  void* ws = with_split ? static_cast<char*>(workspace) + mlp_h_bytes(I, B) : nullptr;
  return gemv_impl(down_packed, down_scales, h, y, H, I, B, &cfg, ws, with_split ? down_ws : 0,
                   Launch{stream});
}

const char* dk_last_error(void) { return dk::g_err.c_str(); }

int dk_abi_version(void) { return DK_ABI_VERSION; }

}  // extern "C"
