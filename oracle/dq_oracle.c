/*
 * dq_oracle.c -- scalar C restatement of the reference's packed-format
 * arithmetic. TEST INFRASTRUCTURE ONLY: linked by tests/ through ctypes as an
 * independent second restatement beside oracle/packer_ref.py (numpy); never
 * part of the product.
 *
 * Follows:
 *   dqo_unpack       dequant/packer.py:164-174   (shift + mask per slot, logical order)
 *   dqo_dequantize   dequant/packer.py:177-189   (fp16_rn((code - off) * scale), fp32 math)
 *   dqo_exact_weight scripts/test_dequant_kernel.py:92-109 (same, no fp16 store)
 *   dqo_gemv_ref     scripts/test_dequant_kernel.py:131-132 (F.linear over exact_weight),
 *                    accumulated in double here, plus |x|@|W|^T for the criterion
 *                    of :112-122.
 *   dqo_f32_to_f16   IEEE 754 binary32 -> binary16, round to nearest even
 *                    (what torch's .to(torch.float16) does on the CPU).
 *
 * Parity pinning: tests/test_oracle.py checks every function here against the
 * golden vectors of tests/golden/packer_golden.npz and against numpy's
 * float16 conversion at every fp16 rounding midpoint.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static const int kInterleave4[8] = {0, 2, 4, 6, 1, 3, 5, 7};
static const int kInterleave2[16] = {0, 4, 8, 12, 1, 5, 9, 13, 2, 6, 10, 14, 3, 7, 11, 15};
static const int kInterleave8[4] = {0, 2, 1, 3};

static const int* slot_order(int bits, int interleaved) {
  static int seq[16] = {0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15};
  if (!interleaved) return seq;
  return bits == 4 ? kInterleave4 : bits == 2 ? kInterleave2 : kInterleave8;
}

static uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float dqo_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t exp = (h >> 10) & 31u, man = h & 1023u;
  if (exp == 0) {
    /* zero or subnormal: man * 2^-24, exact in binary32 */
    float v = (float)man * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  if (exp == 31) return bits_f32(sign | 0x7F800000u | (man << 13));
  return bits_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t dqo_f32_to_f16(float f) {
  uint32_t u = f32_bits(f);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  uint32_t exp = (u >> 23) & 255u, man = u & 0x7FFFFFu;
  if (exp == 255) return (uint16_t)(sign | 0x7C00u | (man ? 0x200u | (man >> 13) : 0u));
  int e = (int)exp - 127 + 15; /* biased binary16 exponent */
  if (e >= 31) return (uint16_t)(sign | 0x7C00u);
  if (e <= 0) {
    /* subnormal (or zero) result: value = full * 2^(e-1-23), quantum 2^-24 */
    if (e < -10) return sign; /* below half the smallest subnormal: rounds to 0 */
    uint32_t full = man | 0x800000u;
    int shift = 14 - e; /* 14..24 */
    uint32_t q = full >> shift, rem = full & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return (uint16_t)(sign | q); /* q may carry into the exponent field: correct */
  }
  uint32_t q = ((uint32_t)e << 10) | (man >> 13), rem = man & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q; /* carry may reach infinity: correct */
  return (uint16_t)(sign | q);
}

void dqo_unpack(const uint32_t* qw, int32_t* out, int64_t n, int64_t k, int bits, int interleaved) {
  const int per = 32 / bits;
  const uint32_t qmax = (1u << bits) - 1u;
  const int* order = slot_order(bits, interleaved);
  const int64_t wpr = k / per;
  for (int64_t r = 0; r < n; ++r)
    for (int64_t w = 0; w < wpr; ++w) {
      uint32_t word = qw[r * wpr + w];
      for (int s = 0; s < per; ++s)
        out[r * k + w * per + order[s]] = (int32_t)((word >> (bits * s)) & qmax);
    }
}

static float code_minus_offset_times_scale(uint32_t code, int64_t r, int64_t g, int64_t ng,
                                           const uint16_t* scales, const uint16_t* zeros,
                                           int bits, int symmetric) {
  float off = symmetric ? (float)(1 << (bits - 1)) : dqo_f16_to_f32(zeros[r * ng + g]);
  volatile float d = (float)code - off; /* fp32 subtract, then a separate fp32 multiply */
  volatile float v = d * dqo_f16_to_f32(scales[r * ng + g]);
  return v;
}

void dqo_exact_weight(const uint32_t* qw, const uint16_t* scales, const uint16_t* zeros,
                      float* out, int64_t n, int64_t k, int bits, int64_t group_size,
                      int symmetric, int interleaved) {
  const int per = 32 / bits;
  const uint32_t qmax = (1u << bits) - 1u;
  const int* order = slot_order(bits, interleaved);
  const int64_t wpr = k / per, ng = k / group_size;
  for (int64_t r = 0; r < n; ++r)
    for (int64_t w = 0; w < wpr; ++w) {
      uint32_t word = qw[r * wpr + w];
      for (int s = 0; s < per; ++s) {
        int64_t col = w * per + order[s];
        out[r * k + col] = code_minus_offset_times_scale((word >> (bits * s)) & qmax, r,
                                                         col / group_size, ng, scales, zeros,
                                                         bits, symmetric);
      }
    }
}

void dqo_dequantize(const uint32_t* qw, const uint16_t* scales, const uint16_t* zeros,
                    uint16_t* out, int64_t n, int64_t k, int bits, int64_t group_size,
                    int symmetric, int interleaved) {
  const int per = 32 / bits;
  const uint32_t qmax = (1u << bits) - 1u;
  const int* order = slot_order(bits, interleaved);
  const int64_t wpr = k / per, ng = k / group_size;
  for (int64_t r = 0; r < n; ++r)
    for (int64_t w = 0; w < wpr; ++w) {
      uint32_t word = qw[r * wpr + w];
      for (int s = 0; s < per; ++s) {
        int64_t col = w * per + order[s];
        out[r * k + col] = dqo_f32_to_f16(code_minus_offset_times_scale(
            (word >> (bits * s)) & qmax, r, col / group_size, ng, scales, zeros, bits, symmetric));
      }
    }
}

/* ref[m, r] = sum_k x[m, k] * w[r, k] and absref = sum_k |x| |w|, in double. */
void dqo_gemv_ref(const uint16_t* x, const float* w, double* ref, double* absref,
                  int64_t m, int64_t n, int64_t k) {
  for (int64_t i = 0; i < m; ++i)
    for (int64_t r = 0; r < n; ++r) {
      double s = 0.0, a = 0.0;
      for (int64_t c = 0; c < k; ++c) {
        double xv = (double)dqo_f16_to_f32(x[i * k + c]);
        double wv = (double)w[r * k + c];
        s += xv * wv;
        a += fabs(xv) * fabs(wv);
      }
      ref[i * n + r] = s;
      absref[i * n + r] = a;
    }
}

/* Convert n fp32 values to fp16 bit patterns (exposed for the rounding test). */
void dqo_f32_to_f16_array(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = dqo_f32_to_f16(in[i]);
}
