// C++ interface of the reference (include/decode_kernel/gemv_w4a16.h:1-51),
// header-only over the C ABI in dk_gemv.h, for C++ callers that used the
// reference's namespace API. Same names, enum values, defaults and argument
// meaning, on HIP types:
//   * cudaStream_t -> hipStream_t, __half from <hip/hip_fp16.h>;
//   * failures throw std::runtime_error carrying dk_last_error() (the
//     reference printed launch errors and continued, csrc/gemv_w4a16.cu:9-16);
//   * w4a16_gemv(..., float* workspace, stream) keeps the reference's
//     workspace contract (gemv_w4a16.h:33): v4 requires the fp32 [B, M]
//     buffer and leaves the fp32 sums of y in it; other versions ignore it
//     (dk_w4a16_gemv_ref_workspace);
//   * w4a16_gemv(..., void* workspace, size_t workspace_bytes, stream) is
//     dk_w4a16_gemv: no version needs a workspace; workspace_bytes() bytes
//     optionally enable the reuse path's split-K tiles.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

#include "decode_kernel/dk_gemv.h"

namespace decode_kernel {

constexpr int kGroupSize = DK_GROUP_SIZE;
constexpr int kNibblesPerWord = DK_NIBBLES_PER_WORD;
constexpr int kWeightsPerInt4 = DK_WEIGHTS_PER_CHUNK;

enum class KernelVersion {
  V0 = DK_V0,  // one thread per row
  V1 = DK_V1,  // one wave64 per row
  V2 = DK_V2,  // 16-byte packed-weight loads
  V3 = DK_V3,  // v2 with the row's scales in LDS
  V4 = DK_V4,  // split-K across the reduction dimension
  V5 = DK_V5,  // tuned streaming kernel
};

struct GemvLaunchConfig {
  KernelVersion version = KernelVersion::V5;
  int split_k = 4;             // used by v4; ignored otherwise
  bool reuse_weights = false;  // MFMA weight-reuse path for batches
  int warps_per_row = 1;       // v1 only: K split across waves of one row
};

namespace detail {

inline dk_gemv_config to_c(const GemvLaunchConfig& cfg) {
  dk_gemv_config c;
  c.version = static_cast<int>(cfg.version);
  c.split_k = cfg.split_k;
  c.reuse_weights = cfg.reuse_weights ? 1 : 0;
  c.warps_per_row = cfg.warps_per_row;
  return c;
}

inline void check(int rc, const char* what) {
  if (rc != DK_OK) throw std::runtime_error(std::string(what) + ": " + dk_last_error());
}

}  // namespace detail

// Device workspace bytes the sized w4a16_gemv overload can take for this
// call: optional, for the reuse path's split-K tiles; 0 otherwise.
inline size_t workspace_bytes(int M, int K, int B, const GemvLaunchConfig& cfg) {
  const dk_gemv_config c = detail::to_c(cfg);
  return dk_gemv_workspace_bytes(M, K, B, &c);
}

// packed:  [M, K/8] uint32, 8 consecutive signed nibbles per word, low first
// scales:  [M, K/128] fp16, symmetric group scale
// x:       [B, K] fp16
// y:       [B, M] fp16
// workspace: fp32 [B, M], required for v4 (as in the reference), which leaves
//            the fp32 sums of y in it; ignored by every other version
inline void w4a16_gemv(const uint32_t* packed, const __half* scales, const __half* x, __half* y,
                       int M, int K, int B, const GemvLaunchConfig& cfg, float* workspace,
                       hipStream_t stream) {
  const dk_gemv_config c = detail::to_c(cfg);
  detail::check(dk_w4a16_gemv_ref_workspace(packed, reinterpret_cast<const uint16_t*>(scales),
                                            reinterpret_cast<const uint16_t*>(x),
                                            reinterpret_cast<uint16_t*>(y), M, K, B, &c, workspace,
                                            stream),
                "w4a16_gemv");
}

// The C ABI's form: `workspace` holds `bytes` >= workspace_bytes() bytes,
// 8-byte aligned, no clearing needed, or is null (for the reuse path null
// runs the single-pass tiles).
inline void w4a16_gemv(const uint32_t* packed, const __half* scales, const __half* x, __half* y,
                       int M, int K, int B, const GemvLaunchConfig& cfg, void* workspace,
                       size_t bytes, hipStream_t stream) {
  const dk_gemv_config c = detail::to_c(cfg);
  detail::check(dk_w4a16_gemv(packed, reinterpret_cast<const uint16_t*>(scales),
                              reinterpret_cast<const uint16_t*>(x), reinterpret_cast<uint16_t*>(y),
                              M, K, B, &c, workspace, bytes, stream),
                "w4a16_gemv");
}

// STREAM-style HBM probes. `partials` is one float per block for the read kernel.
inline void d2d_copy(const void* src, void* dst, size_t bytes, hipStream_t stream) {
  detail::check(dk_d2d_copy(src, dst, bytes, stream), "d2d_copy");
}

inline void stream_read(const void* src, float* partials, size_t bytes, int blocks,
                        hipStream_t stream) {
  detail::check(dk_stream_read(src, partials, bytes, blocks, stream), "stream_read");
}

inline void stream_write(void* dst, size_t bytes, int blocks, hipStream_t stream) {
  detail::check(dk_stream_write(dst, bytes, blocks, stream), "stream_write");
}

inline int stream_recommended_blocks() { return dk_stream_recommended_blocks(); }

// Device stamp written by the GEMV that actually launched. -1 if none.
// Synchronizes the device; reading clears it.
inline int last_kernel_stamp() { return dk_last_kernel_stamp(); }

}  // namespace decode_kernel
