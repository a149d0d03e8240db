/* Llama-style MLP decode step on the W4A16 GEMV (MI355X, gfx950).
 *
 *   h = fp16( silu(Wg x) * (Wu x) )      [B, I]   (dk_gate_up_silu)
 *   y = Wd h                             [B, H]   (the v5 GEMV)
 *
 * Wg, Wu: [I, H] and Wd: [H, I], each in the format of dk_gemv.h (packed
 * int32 [rows, cols/8], fp16 scales [rows, cols/128]); x [B, H] fp16.
 * Gate and up products are accumulated in fp32 (the v5 GEMV's arithmetic)
 * and silu(g) * u is evaluated in fp32 before one rounding to fp16.
 *
 * No counterpart in the reference: it times one GEMV at a time; this is the
 * step either side of its gemv() (python/decode_kernel/__init__.py:32-83)
 * in a decoder MLP, with the gate and up GEMVs fused into one kernel that
 * applies SiLU*mul in its epilogue. Status codes, dk_last_error() and
 * dk_last_kernel_stamp() are those of dk_gemv.h.
 */
#ifndef DECODE_KERNEL_DK_MLP_H_
#define DECODE_KERNEL_DK_MLP_H_

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Dispatch stamp of the fused gate/up kernel (dk_last_kernel_stamp). */
#define DK_STAMP_GATE_UP 20

/* h[b, i] = fp16(silu(g) * u) for g = Wg x, u = Wu x. I, H, B <= 0 is a no-op.
 * H % 128 == 0; gate, up and x 16-byte aligned; scales and h 2-byte aligned. */
int dk_gate_up_silu(const uint32_t* gate_packed, const uint16_t* gate_scales,
                    const uint32_t* up_packed, const uint16_t* up_scales,
                    const uint16_t* x, uint16_t* h, int I, int H, int B,
                    hipStream_t stream);

/* Bytes of workspace dk_mlp_decode takes (0 if empty): h, B * I fp16 padded
 * to 256 bytes, then the down projection's split-K workspace where its
 * batch runs on the split MFMA tiles (dk_gemv_workspace_bytes with
 * reuse_weights). Only the B * I * 2 bytes of h are required; with less than
 * the full size the down projection runs its single-pass tiles. */
size_t dk_mlp_workspace_bytes(int I, int H, int B);

/* y = Wd fp16(silu(Wg x) * (Wu x)): the fused gate/up kernel into the
 * workspace (16-byte aligned, dk_mlp_workspace_bytes), then the GEMV on h
 * (v5 for one row, the weight-reuse path for a batch).
 * H % 128 == 0 and I % 128 == 0. I <= 0 leaves y unwritten (it is zero),
 * as the GEMV does for K = 0; H or B <= 0 is a no-op. */
int dk_mlp_decode(const uint32_t* gate_packed, const uint16_t* gate_scales,
                  const uint32_t* up_packed, const uint16_t* up_scales,
                  const uint32_t* down_packed, const uint16_t* down_scales,
                  const uint16_t* x, uint16_t* y, int I, int H, int B,
                  void* workspace, size_t workspace_bytes, hipStream_t stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* DECODE_KERNEL_DK_MLP_H_ */
