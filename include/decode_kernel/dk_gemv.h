/*
 * decode_kernel C ABI for MI355X (gfx950): W4A16 decode GEMV and HBM probes.
 *
 * Plain C, plain pointers and sizes, no torch types. Every entry point
 * validates its arguments on the host before touching the device and returns
 * a dk_status; dk_last_error() gives the message for the calling thread.
 *
 * Weight format (unchanged from the reference, python/decode_kernel/quantize.py:1-15):
 *   packed  uint32 [M, K/8]   8 signed two's-complement nibbles per word,
 *                             nibble n of word w is weight k = 8*w + n (low first)
 *   scales  fp16   [M, K/128] one symmetric scale per 128-wide K group
 *   x       fp16   [B, K]
 *   y       fp16   [B, M]     y[b,m] = sum_k fp32(scale[m,k/128]) * q[m,k] * fp32(x[b,k])
 * fp16 values travel as their uint16 bit patterns.
 */
#ifndef DECODE_KERNEL_DK_GEMV_H_
#define DECODE_KERNEL_DK_GEMV_H_

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h> /* hipStream_t */

#ifdef __cplusplus
extern "C" {
#endif

/* Format constants. Reference: include/decode_kernel/gemv_w4a16.h:9-11. */
#define DK_GROUP_SIZE 128
#define DK_NIBBLES_PER_WORD 8
#define DK_WEIGHTS_PER_CHUNK 32 /* one 16-byte load of packed weights */

/* Kernel variants. Reference: include/decode_kernel/gemv_w4a16.h:13-20.
 * Each variant is a distinct gfx950 kernel with its own dispatch stamp
 * (dk_last_kernel_stamp): v0..v5 -> 0..5, waves-per-row w (2..8) -> 10+w,
 * weight-reuse -> 15. */
typedef enum dk_kernel_version {
  DK_V0 = 0, /* one thread per row (naive baseline) */
  DK_V1 = 1, /* one wave64 per row, 4-byte coalesced word loads */
  DK_V2 = 2, /* one wave64 per row, 16-byte coalesced loads */
  DK_V3 = 3, /* v2 with the row's group scales staged in LDS */
  DK_V4 = 4, /* split-K: the slices of a row on the waves of one workgroup,
                added in slice order through LDS (one launch, deterministic,
                no workspace) */
  DK_V5 = 5  /* tuned: raw buffer loads (activations first), shape-selected
                rows per wave and activation rows per tile */
} dk_kernel_version;

#define DK_STAMP_REUSE 15
#define DK_STAMP_MULTIWAVE_BASE 10

/* Launch configuration. Reference: include/decode_kernel/gemv_w4a16.h:22-27
 * (GemvLaunchConfig); defaults are the same (v5, split_k 4, no reuse, 1). */
typedef struct dk_gemv_config {
  int version;       /* dk_kernel_version, 0..5 */
  int split_k;       /* v4 only, 1..32: caps the waves that share a row
                        at min(split_k, K/128, 8). With a cap of 1 one
                        wave per row, else two; four (cap >= 4) at
                        M <= 512 on rows of more than 4096 weights and at
                        M <= 1024 on rows of 16384+; two at most for a
                        batch. Ignored otherwise */
  int reuse_weights; /* nonzero: weight-reuse path, ignores version (stamp
                        15). The v5 kernel with batch tiles for up to two
                        batch rows and at M <= 128, up to 32 at M <= 512,
                        up to 11 at M <= 1024, up to 4 at M <= 2048 (8 on
                        rows of fewer than 8192 weights with an odd group
                        count), and at three batch rows unless K >= 8192,
                        M >= 8192, M * K >= 2^27, M >= 3072 with
                        4096 < K < 8192, or 2048 < M <= 4096 with
                        K <= 4096; MFMA tiles otherwise, one workgroup per
                        16 batch rows up to 16 and, above, workgroups of
                        2-8 tiles of 16 batch rows where the groups pair */
  int warps_per_row; /* v1 only, 1..8: wave64s sharing one row's K */
} dk_gemv_config;

typedef enum dk_status {
  DK_OK = 0,
  DK_ERR_INVALID_ARGUMENT = 1, /* rejected on the host; nothing was launched */
  DK_ERR_HIP = 2,              /* the HIP runtime reported an error */
  DK_ERR_UNSUPPORTED = 3       /* valid request beyond a compiled limit */
} dk_status;

/* Fill *cfg with the reference defaults (v5, split_k 4, reuse 0, 1 wave/row). */
void dk_gemv_config_default(dk_gemv_config* cfg);

/* Bytes of device workspace dk_w4a16_gemv takes for this call: 0 for every
 * variant (v4 included) but the weight-reuse path when its MFMA tiles split
 * K over S workgroups per tile (at M <= 1024 where the tiles run, 12 or
 * more batch rows, 33 or more at M <= 512: S = 4 on rows of 28672+ weights
 * with at most 64 tiles of 16 rows x 16 batch rows, S = 2 on rows of
 * 16384+ with at most 64 tiles or 28672+ with at most 128).
 * There it is optional and 8-byte aligned: one 8-byte ticket per tile,
 * padded to 256 bytes, then fp32 partials [S, B, M]; at most 263168 bytes.
 * Without it (NULL or too small) the path runs its single-pass tiles, same
 * results within rounding. It needs no clearing: each ticket carries the
 * call's generation. Calls that overlap in time need separate workspaces.
 * No counterpart in the reference, whose v4 took an fp32 [B, M] buffer
 * zeroed per call (include/decode_kernel/gemv_w4a16.h:33,
 * csrc/bindings.cpp:65-68: see dk_w4a16_gemv_ref_workspace) and whose reuse
 * path took none. Returns 0 for invalid arguments. */
size_t dk_gemv_workspace_bytes(int M, int K, int B, const dk_gemv_config* cfg);

/* Host-side argument check of dk_w4a16_gemv without launching anything
 * (shape rules of csrc/bindings.cpp:10-48). Returns DK_OK or
 * DK_ERR_INVALID_ARGUMENT. */
int dk_gemv_validate(int M, int K, int B, const dk_gemv_config* cfg);

/* y[B, M] = dequant(packed, scales)[M, K] @ x[B, K]^T, asynchronously on
 * `stream`. Replaces decode_kernel::w4a16_gemv
 * (include/decode_kernel/gemv_w4a16.h:34-36, csrc/gemv_w4a16.cu:568-591).
 * M, K or B <= 0 is a no-op returning DK_OK (csrc/gemv_w4a16.cu:571).
 * `workspace` (8-byte aligned) is optional: only the reuse path's split-K
 * tiles use one, of dk_gemv_workspace_bytes() bytes; NULL with 0 is always
 * valid.
 * Differences from the reference: launch errors are returned (the reference
 * printed and continued, csrc/gemv_w4a16.cu:9-16), and split-K is one
 * launch with a deterministic reduction inside the workgroup instead of
 * memset + atomics + convert. */
int dk_w4a16_gemv(const uint32_t* packed, const uint16_t* scales,
                  const uint16_t* x, uint16_t* y, int M, int K, int B,
                  const dk_gemv_config* cfg, void* workspace,
                  size_t workspace_bytes, hipStream_t stream);

/* Size of the per-GPU device array behind dk_w4a16_gemv_noalloc. */
#define DK_NOALLOC_SCRATCH_BYTES ((size_t)512 << 10)

/* dk_w4a16_gemv for callers that cannot allocate: code under HIP graph
 * capture, tight serving loops, hosts that forbid hipMalloc. No counterpart
 * in the reference. The reuse path's split-K tiles take their workspace from
 * a library-owned device array of DK_NOALLOC_SCRATCH_BYTES (512 KiB) on each
 * GPU, held until the process ends; nothing is allocated, cleared or freed
 * by a call. Every call's dk_gemv_workspace_bytes() fits it (at most 263168
 * bytes); one that did not would return DK_ERR_UNSUPPORTED before any
 * launch. Every call on one GPU shares
 * that GPU's array: calls that overlap in time on one GPU (different
 * streams, or host threads) race and must not be issued. Arguments, checks
 * and results otherwise as dk_w4a16_gemv. */
int dk_w4a16_gemv_noalloc(const uint32_t* packed, const uint16_t* scales, const uint16_t* x,
                          uint16_t* y, int M, int K, int B, const dk_gemv_config* cfg,
                          hipStream_t stream);

/* dk_w4a16_gemv with the reference's workspace contract, for callers written
 * against decode_kernel::w4a16_gemv (include/decode_kernel/gemv_w4a16.h:29-36,
 * csrc/gemv_w4a16.cu:474-481): for v4, `workspace` is the caller's fp32
 * [B, M] buffer (required, as in the reference), which holds the fp32 sums
 * of y after the call, as the reference's did; nothing past it is touched.
 * Every other variant ignores `workspace` and runs as dk_w4a16_gemv with
 * none. */
int dk_w4a16_gemv_ref_workspace(const uint32_t* packed, const uint16_t* scales,
                                const uint16_t* x, uint16_t* y, int M, int K, int B,
                                const dk_gemv_config* cfg, float* workspace,
                                hipStream_t stream);

/* The kernel dk_w4a16_gemv would launch for this call, without launching
 * anything or touching a device: its demangled name (as a rocprofv3 kernel
 * trace prints it), grid and workgroup size, and the number of launches the
 * call makes. `workspace_bytes` is what the call would pass (it selects the
 * reuse path's split-K tiles). No counterpart in the reference; it lets a
 * benchmark or profile name the kernel behind a measurement. */
typedef struct dk_launch_info {
  char kernel[512];
  unsigned grid[3];
  unsigned block[3];
  int launches;
} dk_launch_info;

int dk_gemv_describe(int M, int K, int B, const dk_gemv_config* cfg, size_t workspace_bytes,
                     dk_launch_info* info);

/* Kernel-native "paired" weight layout: the same two's-complement int4
 * nibbles and scales, with each word's nibbles permuted so that q_{2j} is at
 * bits 4j..4j+3 and q_{2j+1} at bits 16+4j..19+4j (j = 0..3). The decode
 * then yields the natural activation pairs (x_{2j}, x_{2j+1}), so the GEMV
 * skips the activation pairing permutes. Scales are unchanged. An offline
 * repack of packed [M, K/8]; dk_unpack_paired inverts it bit for bit.
 * No counterpart in the reference, whose format (quantize.py:1-15) is the
 * API format here too. */
#define DK_STAMP_PAIRED 25

int dk_repack_paired(const uint32_t* packed, uint32_t* paired, int M, int K,
                     hipStream_t stream);
int dk_unpack_paired(const uint32_t* paired, uint32_t* packed, int M, int K,
                     hipStream_t stream);

/* The v5 GEMV on paired weights (stamp DK_STAMP_PAIRED); arguments, checks
 * and results as dk_w4a16_gemv with the default configuration (a batch runs
 * the v5 kernel's batch tiles; the weight-reuse MFMA tiles read the API
 * layout only). */
int dk_w4a16_gemv_paired(const uint32_t* paired, const uint16_t* scales,
                         const uint16_t* x, uint16_t* y, int M, int K, int B,
                         hipStream_t stream);

/* Quantize fp32 W[M, K] (row-major, 16-byte aligned) into the format above:
 * packed [M, K/8] and fp16 scales [M, K/128], bit-exact with the reference
 * quantizer on fp32 input: per 128-group scale = max(amax/7, 1e-8) in fp32,
 * q = clamp(round_half_even(w/scale), -7, 7), scale stored as fp16 (RNE).
 * Replaces quantize_and_pack on device tensors
 * (python/decode_kernel/quantize.py:26-51). Inputs must be finite. */
int dk_quantize_pack_f32(const float* w, int M, int K, uint32_t* packed,
                         uint16_t* scales, hipStream_t stream);

/* STREAM probes. Reference: include/decode_kernel/gemv_w4a16.h:38-43,
 * csrc/gemv_w4a16.cu:593-626. `bytes` must be a multiple of 16.
 * dk_stream_read writes one fp32 partial sum per block into `partials`
 * (blocks entries); blocks < 1 selects dk_stream_recommended_blocks(). */
int dk_d2d_copy(const void* src, void* dst, size_t bytes, hipStream_t stream);
int dk_stream_read(const void* src, float* partials, size_t bytes, int blocks,
                   hipStream_t stream);
int dk_stream_write(void* dst, size_t bytes, int blocks, hipStream_t stream);

/* Block count for the probes on the current device: CUs*32 clamped to
 * [1024, 8192] (csrc/gemv_w4a16.cu:602-609 queried device 0 instead).
 * Returns a negative dk_status on error. */
int dk_stream_recommended_blocks(void);

/* Stamp of the last GEMV kernel launched on the current device, or -1 if
 * none was launched since the previous read. The host records it when a
 * launch succeeds (the reference's kernels wrote it to a device global,
 * cleared with an extra host-to-device copy before every launch,
 * csrc/gemv_w4a16.cu:18-25,553-564,573; that store costs 0.04-0.05 us per
 * launch here). Synchronises the device, then reads the stamp and clears it
 * to -1. Returns -1 on error as well; see dk_last_error(). */
int dk_last_kernel_stamp(void);

/* An empty kernel on `stream`: the per-launch floor for the benchmark.
 * No counterpart in the reference. */
int dk_empty_kernel(hipStream_t stream);

/* Message for the last non-DK_OK status returned on the calling thread. */
const char* dk_last_error(void);

/* ABI version of this header, (major << 16) | minor. */
int dk_abi_version(void);
#define DK_ABI_VERSION ((1 << 16) | 4)

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* DECODE_KERNEL_DK_GEMV_H_ */
