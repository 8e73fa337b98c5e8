// Bit-exact restatement of the reference quantizer's arithmetic.
//
// The reference quantizes in the *source* dtype, one torch op at a time
// (reference src/dart/quantization.py:179-186, src/dart/mixed.py:201-209).
// Each bf16/fp16 op computes in fp32 and rounds the result to the storage
// dtype with round-to-nearest-even; fp32 inputs stay in fp32.  The helpers
// here replay that sequence with explicit rounding after every op so that the
// GPU kernels produce the same codes, scales and zero points.
//
//   range = rnd(max - min)                    quantization.py:184
//   range = max(range, rnd(eps))              eps 1e-4 (half types) / 1e-6 (fp32)
//   scale = rnd(range / qmax)                 true division
//   code  = clamp(rint(rnd(rnd(x - min) / scale)), 0, qmax)   :185-186
//   scale_meta = cast(scale), zero_meta = cast(min)           :194-195
//
// Dequantization (quantization.py:103-106, mixed.py:90-94) is
//   value = to_out( rnd_meta( rnd_meta(code * scale) + zero ) ).
//
// Token means used for channel selection follow ATen's CPU reduction:
// fp32 accumulation with a 4-level cascade (level step 2^max(4, ceil(log2 n)/4)),
// then one fp32 division by n and one rounding to the source dtype.
#pragma once
#include <stdint.h>
#include <string.h>

#ifndef DKV_HD
#if defined(__HIPCC__)
#define DKV_HD __host__ __device__
#else
#define DKV_HD
#endif
#endif

namespace dkv {

// Element types shared with the C ABI (values match DKV_DTYPE_* in dartkv.h).
enum DType : int32_t { kF32 = 0, kF16 = 1, kBF16 = 2, kF64 = 3, kU8 = 4, kI32 = 5 };

DKV_HD inline uint32_t f2u(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  return u;
}
DKV_HD inline float u2f(uint32_t u) {
  float x;
  memcpy(&x, &u, 4);
  return x;
}

// ---- bf16 ----
DKV_HD inline uint16_t bf16_bits_rne(float x) {
  uint32_t u = f2u(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
DKV_HD inline float bf16_to_f32(uint16_t b) { return u2f(((uint32_t)b) << 16); }
DKV_HD inline float round_bf16(float x) { return bf16_to_f32(bf16_bits_rne(x)); }

// ---- fp16 (IEEE binary16), software conversions that handle subnormals ----
DKV_HD inline uint16_t f16_bits_rne(float x) {
  uint32_t u = f2u(x);
  const uint32_t sign = (u >> 16) & 0x8000u;
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);       // NaN
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);      // rounds to inf (>= 65520)
  if (a < 0x38800000u) {                                        // below 2^-14: subnormal or zero
    if (a < 0x33000000u) return (uint16_t)sign;                 // < 2^-25 rounds to 0 (2^-25 ties to 0)
    const uint32_t exp = a >> 23;                               // 102..112
    const uint32_t mant = (a & 0x7fffffu) | 0x800000u;          // 24-bit significand
    const uint32_t shift = 126u - exp;                          // value = mant * 2^(exp-150); unit 2^-24
    uint32_t q = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return (uint16_t)(sign | q);
  }
  // normal: rebias exponent (127 -> 15) and round 23-bit mantissa to 10 bits
  uint32_t r = a - 0x38000000u;                                 // exponent - 112
  r += 0xfffu + ((r >> 13) & 1u);
  return (uint16_t)(sign | (r >> 13));
}
DKV_HD inline float f16_to_f32(uint16_t h) {
  const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu;
  uint32_t m = h & 0x3ffu;
  if (e == 0) {
    if (m == 0) return u2f(sign);
    // subnormal: m * 2^-24
    float v = (float)m * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
  return u2f(sign | ((e + 112u) << 23) | (m << 13));
}
DKV_HD inline float round_f16(float x) { return f16_to_f32(f16_bits_rne(x)); }

// Round an fp32 value to the storage precision of `dt` (fp32 is identity).
DKV_HD inline float round_to(float x, int dt) {
  if (dt == kBF16) return round_bf16(x);
  if (dt == kF16) return round_f16(x);
  return x;
}

// eps used by the reference clamp, already rounded to the source dtype.
DKV_HD inline float quant_eps(int dt) {
  if (dt == kBF16) return round_bf16(1.0e-4f);
  if (dt == kF16) return round_f16(1.0e-4f);
  return 1.0e-6f;
}

// Round-half-to-even of a non-negative float (torch.round semantics).
DKV_HD inline float rint_even(float x) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_rintf(x);
#else
  return __builtin_rintf(x);
#endif
}

// scale for one group, in the source dtype's precision.
DKV_HD inline float group_scale(float mn, float mx, float qmax, int dt) {
  float range = round_to(mx - mn, dt);
  const float eps = quant_eps(dt);
  if (!(range >= eps)) range = eps;
  return round_to(range / qmax, dt);
}

// code for one element given the group's min and scale (source dtype values).
DKV_HD inline uint32_t group_code(float x, float mn, float scale, float qmax, int dt) {
  const float diff = round_to(x - mn, dt);
  const float q = rint_even(round_to(diff / scale, dt));
  float c = q < 0.0f ? 0.0f : q;
  c = c > qmax ? qmax : c;
  return (uint32_t)c;
}

// Convert a source-dtype value to the metadata dtype and store it.
DKV_HD inline void store_meta(void* base, int64_t index, float v, int meta) {
  if (meta == kF16) {
    ((uint16_t*)base)[index] = f16_bits_rne(v);
  } else if (meta == kBF16) {
    ((uint16_t*)base)[index] = bf16_bits_rne(v);
  } else if (meta == kF32) {
    ((float*)base)[index] = v;
  } else {
    ((double*)base)[index] = (double)v;
  }
}

DKV_HD inline double load_meta(const void* base, int64_t index, int meta) {
  if (meta == kF16) return (double)f16_to_f32(((const uint16_t*)base)[index]);
  if (meta == kBF16) return (double)bf16_to_f32(((const uint16_t*)base)[index]);
  if (meta == kF32) return (double)((const float*)base)[index];
  return ((const double*)base)[index];
}

// The reference dequantization chain for one element, returned as the fp32
// value the attention oracle consumes (`.float()` of the cache-dtype tensor).
DKV_HD inline float dequant_value(uint32_t code, double scale, double zero, int meta, int out_dt) {
  if (meta == kF64) {
    const double v = (double)code * scale + 0.0;
    const double w = v + zero;
    // double -> float (RNE) then float -> out dtype (RNE), as c10 converts.
    return round_to((float)w, out_dt);
  }
  const float s = (float)scale, z = (float)zero;
  const float prod = round_to((float)code * s, meta);
  const float sum = round_to(prod + z, meta);
  return round_to(sum, out_dt);
}

DKV_HD inline float load_elem(const void* base, int64_t index, int dt) {
  if (dt == kBF16) return bf16_to_f32(((const uint16_t*)base)[index]);
  if (dt == kF16) return f16_to_f32(((const uint16_t*)base)[index]);
  return ((const float*)base)[index];
}

// ATen CPU cascade-sum order for n rows: returns the level step exponent.
DKV_HD inline int cascade_level_power(int64_t n) {
  int ceil_log2 = 0;
  while (((int64_t)1 << ceil_log2) < n) ++ceil_log2;
  const int p = ceil_log2 / 4;
  return p > 4 ? p : 4;
}

}  // namespace dkv
