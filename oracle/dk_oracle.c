/*
 * Scalar C restatement of the W4A16 format and GEMV, written independently of
 * oracle/oracle.py so each can catch the other's mistakes.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ (through oracle/c_oracle.py) as a
 * checker. Nothing in the product links or calls it.
 *
 *   dko_quantize_pack  python/decode_kernel/quantize.py:26-51 (per element,
 *                      fp32 arithmetic, round-half-even, hand-written fp16 RNE)
 *   dko_unpack         python/decode_kernel/quantize.py:54-63 and the nibble
 *                      decode of csrc/gemv_w4a16.cu:27-29
 *   dko_gemv_f64       python/decode_kernel/reference.py:17-26 in float64
 *   dko_f32_to_f16 / dko_f16_to_f32   IEEE-754 binary16 conversions (RNE)
 *
 * Build: make -C oracle   (gcc, no fast-math: IEEE fp32 division and rint).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define DKO_GROUP 128

uint16_t dko_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, sizeof x);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
  if (ax < 0x38800000u) {                                     /* below 2^-14: fp16 subnormal */
    const int e = (int)(ax >> 23);                            /* biased fp32 exponent */
    const uint32_t sig = (ax & 0x7fffffu) | (e ? 0x800000u : 0u);
    const int exp2 = (e ? e : 1) - 127 - 23;                  /* value = sig * 2^exp2 */
    const int s = -(exp2 + 24);                               /* m = sig * 2^(exp2+24) */
    if (s >= 32) return (uint16_t)sign;
    uint32_t m = sig >> s;
    const uint32_t rem = sig & ((1u << s) - 1u);
    const uint32_t half = 1u << (s - 1);
    if (rem > half || (rem == half && (m & 1u))) m += 1u;
    return (uint16_t)(sign | m);
  }
  const uint32_t e16 = (ax >> 23) - 127u + 15u;
  const uint32_t mant = ax & 0x7fffffu;
  uint32_t h = (e16 << 10) | (mant >> 13);
  const uint32_t rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
  return (uint16_t)(sign | h);
}

float dko_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu;
  const uint32_t m = h & 0x3ffu;
  float v;
  if (e == 0) {
    v = ldexpf((float)m, -24);
  } else if (e == 31) {
    uint32_t bits = 0x7f800000u | (m << 13);
    memcpy(&v, &bits, sizeof v);
  } else {
    uint32_t bits = ((e - 15u + 127u) << 23) | (m << 13);
    memcpy(&v, &bits, sizeof v);
  }
  uint32_t out;
  memcpy(&out, &v, sizeof out);
  out |= sign;
  memcpy(&v, &out, sizeof v);
  return v;
}

/* Returns 0 on success, -1 if K is not a multiple of 128. */
int dko_quantize_pack(const float* w, int64_t M, int64_t K, int32_t* packed, uint16_t* scales) {
  if (K % DKO_GROUP != 0) return -1;
  const int64_t G = K / DKO_GROUP;
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t g = 0; g < G; ++g) {
      const float* src = w + m * K + g * DKO_GROUP;
      float amax = 0.0f;
      for (int i = 0; i < DKO_GROUP; ++i) {
        const float a = fabsf(src[i]);
        if (a > amax) amax = a;
      }
      float scale = amax / 7.0f;
      const float floor_ = 1e-8f;
      if (scale < floor_) scale = floor_;
      scales[m * G + g] = dko_f32_to_f16(scale);
      for (int i = 0; i < DKO_GROUP; ++i) {
        float r = rintf(src[i] / scale); /* default rounding mode: nearest, ties to even */
        if (r < -7.0f) r = -7.0f;
        if (r > 7.0f) r = 7.0f;
        const int q = (int)r;
        const int64_t k = g * DKO_GROUP + i;
        uint32_t* word = (uint32_t*)&packed[m * (K / 8) + k / 8];
        if (k % 8 == 0) *word = 0u;
        *word |= ((uint32_t)q & 0xFu) << (4 * (k % 8));
      }
    }
  }
  return 0;
}

void dko_unpack(const int32_t* packed, int64_t M, int64_t K, int32_t* q) {
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t k = 0; k < K; ++k) {
      const uint32_t word = (uint32_t)packed[m * (K / 8) + k / 8];
      const int nib = (int)((word >> (4 * (k % 8))) & 0xFu);
      q[m * K + k] = nib >= 8 ? nib - 16 : nib;
    }
  }
}

/* y[b*M + m] = sum_k double(scale[m, k/128]) * q[m,k] * double(x[b*K + k]). */
void dko_gemv_f64(const int32_t* packed, const uint16_t* scales, const uint16_t* x, int64_t M,
                  int64_t K, int64_t B, double* y) {
  const int64_t G = K / DKO_GROUP;
  for (int64_t b = 0; b < B; ++b) {
    for (int64_t m = 0; m < M; ++m) {
      double acc = 0.0;
      for (int64_t k = 0; k < K; ++k) {
        const uint32_t word = (uint32_t)packed[m * (K / 8) + k / 8];
        const int nib = (int)((word >> (4 * (k % 8))) & 0xFu);
        const int qv = nib >= 8 ? nib - 16 : nib;
        const double s = (double)dko_f16_to_f32(scales[m * G + k / DKO_GROUP]);
        acc += s * (double)qv * (double)dko_f16_to_f32(x[b * K + k]);
      }
      y[b * M + m] = acc;
    }
  }
}
