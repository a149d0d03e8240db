// Device-side building blocks shared by the gfx950 W4A16 GEMV kernels.
//
// Nibble decode. The reference decodes one signed nibble at a time with two
// shifts and an int->float convert per weight (csrc/gemv_w4a16.cu:27-39).
// Here a whole 32-bit word (8 weights) is decoded into four packed fp16 pairs
// with the IEEE-754 binary16 exponent trick: OR an offset-binary nibble u
// (0..15) into the mantissa of 1024.0 (0x6400) to get the fp16 value 1024+u,
// then subtract 1032 to get q = u - 8 exactly. Two nibbles 16 bits apart are
// decoded by one AND/XOR, so a word costs one shift, four AND/XOR (each one
// v_bitop3_b32 on gfx950) and four packed fp16 ops: about 1.1 VALU
// operations per weight, and every step is exact.
//
// The pairs come out as (q0,q4), (q1,q5), (q2,q6), (q3,q7). Activations are
// paired the same way with v_perm_b32, once per 16-byte chunk of x, and the
// pair products are summed with v_dot2_f32_f16 (fp16 x fp16 products are
// exact in fp32; accumulation is fp32).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dk {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

constexpr int kGroupSize = 128;
constexpr int kWave = 64;

__device__ __forceinline__ h2_t as_h2(uint32_t v) { return __builtin_bit_cast(h2_t, v); }

// Decode the 8 signed nibbles of `w` (nibble n = bits 4n..4n+3, two's
// complement, reference layout include/decode_kernel/gemv_w4a16.h:29-30)
// into q[j] = (q_j, q_{j+4}) for j = 0..3.
//
// The two's-complement -> offset-binary flip (XOR of the nibble's top bit)
// and the OR of the 0x6400 exponent are one XOR with a constant after the
// mask: (w & M) ^ (0x6400.. | sign bits inside M). AND-then-XOR is a single
// v_bitop3_b32, so a pair costs one logic op and one packed fp16 op.
__device__ __forceinline__ void unpack_word(uint32_t w, h2_t (&q)[4]) {
  const uint32_t v = w >> 8;
  const h2_t sub = {(_Float16)-1032.0f, (_Float16)-1032.0f};
  const h2_t sixteenth = {(_Float16)0.0625f, (_Float16)0.0625f};
  const h2_t sub16 = {(_Float16)-72.0f, (_Float16)-72.0f};
  // Low nibble of each 16-bit half: fp16 1024 + u, u = nibble ^ 8.
  q[0] = as_h2((w & 0x000F000Fu) ^ 0x64086408u) + sub;
  q[2] = as_h2((v & 0x000F000Fu) ^ 0x64086408u) + sub;
  // Second nibble of each half lands in mantissa bits 4..7: 1024 + 16u,
  // and (1024 + 16u)/16 - 72 = u - 8.
  q[1] = as_h2((w & 0x00F000F0u) ^ 0x64806480u) * sixteenth + sub16;
  q[3] = as_h2((v & 0x00F000F0u) ^ 0x64806480u) * sixteenth + sub16;
}

// The kernel-native "paired" layout (an offline repack of the format above,
// dk_repack_paired) permutes each word's two's-complement nibbles so that
// q_{2j} sits at bits 4j..4j+3 and q_{2j+1} at bits 16+4j..19+4j. The same
// unpack_word then yields (q0,q1), (q2,q3), (q4,q5), (q6,q7): the natural
// fp16 pairs of eight consecutive activations, which need no v_perm.

// Pair eight consecutive fp16 activations (one 16-byte load: .x=(x0,x1),
// .y=(x2,x3), .z=(x4,x5), .w=(x6,x7)) to match unpack_word's order.
__device__ __forceinline__ void pair_x(const uint4& xv, h2_t (&p)[4]) {
  p[0] = as_h2(__builtin_amdgcn_perm(xv.z, xv.x, 0x05040100u));  // (x0, x4)
  p[1] = as_h2(__builtin_amdgcn_perm(xv.z, xv.x, 0x07060302u));  // (x1, x5)
  p[2] = as_h2(__builtin_amdgcn_perm(xv.w, xv.y, 0x05040100u));  // (x2, x6)
  p[3] = as_h2(__builtin_amdgcn_perm(xv.w, xv.y, 0x07060302u));  // (x3, x7)
}

// sum_{n<8} q_n * x_n for one packed word, accumulated into `acc` in fp32.
__device__ __forceinline__ float dot_word(uint32_t w, const h2_t (&xp)[4], float acc) {
  h2_t q[4];
  unpack_word(w, q);
  acc = __builtin_amdgcn_fdot2(q[0], xp[0], acc, false);
  acc = __builtin_amdgcn_fdot2(q[1], xp[1], acc, false);
  acc = __builtin_amdgcn_fdot2(q[2], xp[2], acc, false);
  acc = __builtin_amdgcn_fdot2(q[3], xp[3], acc, false);
  return acc;
}

// Eight decoded weights of one word in MFMA operand order
// [q0,q4,q1,q5,q2,q6,q3,q7]; pair_x8 gives activations in the same order.
__device__ __forceinline__ h8_t unpack_word_h8(uint32_t w) {
  h2_t q[4];
  unpack_word(w, q);
  h8_t r;
  r[0] = q[0][0]; r[1] = q[0][1]; r[2] = q[1][0]; r[3] = q[1][1];
  r[4] = q[2][0]; r[5] = q[2][1]; r[6] = q[3][0]; r[7] = q[3][1];
  return r;
}

__device__ __forceinline__ h8_t pair_x8(const uint4& xv) {
  h2_t p[4];
  pair_x(xv, p);
  h8_t r;
  r[0] = p[0][0]; r[1] = p[0][1]; r[2] = p[1][0]; r[3] = p[1][1];
  r[4] = p[2][0]; r[5] = p[2][1]; r[6] = p[3][0]; r[7] = p[3][1];
  return r;
}

// Weight layouts the streaming kernels read: how a word decodes and how
// eight activations are paired to match it.
struct LayoutLogical {
  static constexpr int kStamp = 5;
  static __device__ __forceinline__ void unpack(uint32_t w, h2_t (&q)[4]) { unpack_word(w, q); }
  static __device__ __forceinline__ void pair(const uint4& xv, h2_t (&p)[4]) { pair_x(xv, p); }
};
struct LayoutPaired {
  static constexpr int kStamp = 25;
  static __device__ __forceinline__ void unpack(uint32_t w, h2_t (&q)[4]) { unpack_word(w, q); }
  static __device__ __forceinline__ void pair(const uint4& xv, h2_t (&p)[4]) {
    p[0] = as_h2(xv.x);  // (x0, x1)
    p[1] = as_h2(xv.y);  // (x2, x3)
    p[2] = as_h2(xv.z);  // (x4, x5)
    p[3] = as_h2(xv.w);  // (x6, x7)
  }
};

template <int kCtrl, int kRowMask = 0xF>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, kRowMask, 0xF, false));
}

// Sum over the 64 lanes of a wave with DPP only (no LDS traffic). The total
// is valid in lanes 48..63; lane 63 is the one callers read.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<0xB1>(v);        // quad_perm [1,0,3,2]: pairs
  v += dpp<0x4E>(v);        // quad_perm [2,3,0,1]: quads
  v += dpp<0x141>(v);       // row_half_mirror: 8 lanes
  v += dpp<0x140>(v);       // row_mirror: 16-lane rows
  v += dpp<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
  v += dpp<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
  return v;
}

// Workgroups are dealt to the 8 XCDs of an MI355X round-robin (workgroup i
// to XCD i % 8). Renumber them so XCD x handles one contiguous range of
// workgroup ids: a bijection on [0, n) for any n, so correctness does not
// depend on the dealing order; it only changes which XCD streams which rows.
__device__ __forceinline__ int xcd_contiguous_block(int wg, int n) {
  const int q = n >> 3, r = n & 7, x = wg & 7;
  return x * q + (x < r ? x : r) + (wg >> 3);
}

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

__device__ __forceinline__ uint4 zero4() { return make_uint4(0u, 0u, 0u, 0u); }

}  // namespace dk
