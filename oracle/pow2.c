/* C restatement of tbf16's bit-level hot-path arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ through ctypes as a second,
 * independent route to the exponents and the rounded payloads that the HIP
 * kernels must reproduce bit for bit. Nothing in the product links it.
 *
 * Restated from the reference (paths relative to tech-cosmos/turing-bf16):
 *   pow2_exp        tbf16/csrc/small_kernels.cu:12-18   (clamped scale exponent)
 *   pow2_exp_fused  tbf16/csrc/gemm_sm75.cu:19-23       (upper clamp only)
 *   scaled_f16      small_kernels.cu:68-69, gemm_sm75.cu:72-75
 *                   (__floats2half2_rn of x * 2^p: round to nearest even)
 *   f32_to_bf16     small_kernels.cu:99, gemm_sm75.cu:215 (__floats2bfloat162_rn)
 * The rounding is written from the IEEE-754 definition, not from any library.
 */
#include <stdint.h>
#include <string.h>

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

static int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }

int tbf16o_pow2_exp(float amax, int t) {
  int e = clampi((int)((f2u(amax) >> 23) & 0xFF), 1, 252);
  int se = clampi(253 + t - e, 1, 254);
  return se - 127;
}

int tbf16o_pow2_exp_fused(float amax, int t) {
  int e = clampi((int)((f2u(amax) >> 23) & 0xFF), 1, 252);
  int se = 253 + t - e;
  if (se > 254) se = 254;
  return se - 127;
}

/* fp32 -> fp16 bits, round to nearest even, with subnormals, overflow to inf
 * and NaN kept quiet. */
uint16_t tbf16o_f32_to_f16(float f) {
  uint32_t u = f2u(f);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  uint32_t ex = (u >> 23) & 0xFF, man = u & 0x7FFFFFu;
  if (ex == 0xFF) return (uint16_t)(sign | 0x7C00u | (man ? 0x200u | (man >> 13) : 0));
  int e = (int)ex - 127;            /* unbiased exponent */
  if (ex == 0) return sign;         /* fp32 subnormals are far below fp16's range */
  uint32_t sig = man | 0x800000u;   /* 24-bit significand, value = sig * 2^(e-23) */
  int shift;                        /* bits to drop from sig */
  uint32_t hexp;
  if (e >= -14) {                   /* normal fp16: keep 11 bits */
    shift = 13;
    hexp = (uint32_t)(e + 15);
  } else {                          /* subnormal fp16: value = q * 2^-24 */
    shift = 13 + (-14 - e);
    hexp = 0;
    if (shift > 25) return sign;    /* below half of the smallest subnormal */
  }
  uint32_t q = sig >> shift;
  uint32_t rem = sig & ((1u << shift) - 1u), half = 1u << (shift - 1);
  if (rem > half || (rem == half && (q & 1u))) q += 1;
  uint32_t bits;
  if (hexp == 0) {
    bits = q;                       /* may carry into the smallest normal: correct */
  } else {
    if (q == 0x800u) { q = 0x400u; hexp += 1; }  /* significand overflow */
    if (hexp >= 31) return (uint16_t)(sign | 0x7C00u);
    bits = (hexp << 10) | (q & 0x3FFu);
  }
  return (uint16_t)(sign | bits);
}

uint16_t tbf16o_f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* fp16(bf16 * 2^p): the scaled conversion of quantize_rows / the fused GEMM. The
 * product is formed in fp32 exactly like the reference (x * s with s = 2^p). */
uint16_t tbf16o_scaled_f16(uint16_t bf16_bits, int p) {
  float x = u2f((uint32_t)bf16_bits << 16);
  float s = u2f((uint32_t)(p + 127) << 23);  /* p in [-126, 127] */
  return tbf16o_f32_to_f16(x * s);
}

void tbf16o_pow2_exp_n(const float* amax, int64_t n, int t, int fused, int32_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = fused ? tbf16o_pow2_exp_fused(amax[i], t) : tbf16o_pow2_exp(amax[i], t);
}

void tbf16o_scaled_f16_n(const uint16_t* bf16_bits, int64_t n, int p, uint16_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = tbf16o_scaled_f16(bf16_bits[i], p);
}

void tbf16o_f32_to_bf16_n(const float* x, int64_t n, uint16_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = tbf16o_f32_to_bf16(x[i]);
}

void tbf16o_f32_to_f16_n(const float* x, int64_t n, uint16_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = tbf16o_f32_to_f16(x[i]);
}
