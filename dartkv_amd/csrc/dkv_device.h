// Device-side helpers shared by the DartKV HIP kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dkv_numeric.h"

namespace dkv {

// Hardware conversions that give the same results as the software ones in
// dkv_numeric.h (IEEE round-to-nearest-even, fp16 subnormals preserved).
__device__ __forceinline__ float dev_round_f16(float x) { return (float)(_Float16)x; }

__device__ __forceinline__ float dev_round_to(float x, int dt) {
  if (dt == kBF16) return round_bf16(x);
  if (dt == kF16) return dev_round_f16(x);
  return x;
}

// Element `index` of `base` (dtype dt) as fp32; a float64 element is rounded
// to nearest, as torch's `.float()` does (the reference's attention computes
// in fp32 for every cache dtype, attention.py:62-77).
__device__ __forceinline__ float dev_load(const void* base, int64_t index, int dt) {
  if (dt == kBF16) return bf16_to_f32(((const uint16_t*)base)[index]);
  if (dt == kF16) return (float)(((const _Float16*)base)[index]);
  if (dt == kF64) return (float)((const double*)base)[index];
  return ((const float*)base)[index];
}

// x[r] = element idx(r) of `base` (dtype dt) as fp32 for r < N, or 0 where
// idx(r) < 0 (element 0 is read there, so base must hold at least one
// element).  The dtype is tested once and every load is unconditional, so all
// N loads are issued before the first wait (a per-element dtype switch or a
// per-lane branch makes the compiler wait for each load in turn).
template <int N, typename IndexFn>
__device__ __forceinline__ void dev_load_n(const void* base, int dt, float (&x)[N], IndexFn idx) {
  int64_t at[N];
#pragma unroll
  for (int r = 0; r < N; ++r) at[r] = idx(r);
  if (dt == kBF16 || dt == kF16) {
    uint16_t raw[N];
#pragma unroll
    for (int r = 0; r < N; ++r) raw[r] = ((const uint16_t*)base)[at[r] >= 0 ? at[r] : 0];
#pragma unroll
    for (int r = 0; r < N; ++r) {
      const float v = dt == kBF16 ? bf16_to_f32(raw[r]) : (float)__builtin_bit_cast(_Float16, raw[r]);
      x[r] = at[r] >= 0 ? v : 0.f;
    }
  } else if (dt == kF64) {
#pragma unroll
    for (int r = 0; r < N; ++r) {
      const float v = (float)((const double*)base)[at[r] >= 0 ? at[r] : 0];
      x[r] = at[r] >= 0 ? v : 0.f;
    }
  } else {
#pragma unroll
    for (int r = 0; r < N; ++r) {
      const float v = ((const float*)base)[at[r] >= 0 ? at[r] : 0];
      x[r] = at[r] >= 0 ? v : 0.f;
    }
  }
}

__device__ __forceinline__ void dev_store(void* base, int64_t index, float v, int dt) {
  if (dt == kBF16) {
    ((uint16_t*)base)[index] = bf16_bits_rne(v);
  } else if (dt == kF16) {
    ((_Float16*)base)[index] = (_Float16)v;
  } else if (dt == kF64) {
    ((double*)base)[index] = (double)v;
  } else {
    ((float*)base)[index] = v;
  }
}

__device__ __forceinline__ void dev_store_meta(void* base, int64_t index, float v, int meta) {
  if (meta == kF16) {
    ((_Float16*)base)[index] = (_Float16)v;
  } else if (meta == kBF16) {
    ((uint16_t*)base)[index] = bf16_bits_rne(v);
  } else if (meta == kF32) {
    ((float*)base)[index] = v;
  } else {
    ((double*)base)[index] = (double)v;
  }
}

// A float64 value (scale or minimum of an fp64 source) in the metadata dtype:
// exact for float64; otherwise rounded to fp32 first, then to the 16-bit type,
// which is how torch converts float64 to float16 / bfloat16 (through float).
__device__ __forceinline__ void dev_store_meta(void* base, int64_t index, double v, int meta) {
  if (meta == kF64) {
    ((double*)base)[index] = v;
  } else {
    dev_store_meta(base, index, (float)v, meta);
  }
}

__device__ __forceinline__ double dev_load_meta(const void* base, int64_t index, int meta) {
  if (meta == kF16) return (double)(float)(((const _Float16*)base)[index]);
  if (meta == kBF16) return (double)bf16_to_f32(((const uint16_t*)base)[index]);
  if (meta == kF32) return (double)((const float*)base)[index];
  return ((const double*)base)[index];
}

// Reference dequantization chain (quantization.py:103-106): meta-dtype
// multiply, meta-dtype add, cast to the cache dtype; returned as fp32.
__device__ __forceinline__ float dev_dequant(uint32_t code, double scale, double zero, int meta, int out_dt) {
  if (meta == kF64) {
    const double w = __dadd_rn(__dmul_rn((double)code, scale), zero);
    return dev_round_to((float)w, out_dt);
  }
  const float s = (float)scale, z = (float)zero;
  const float prod = dev_round_to(__fmul_rn((float)code, s), meta);
  const float sum = dev_round_to(__fadd_rn(prod, z), meta);
  return dev_round_to(sum, out_dt);
}

// The dequantized value written to `out` (dtype out_dt): dev_dequant's chain,
// except that float64 metadata into a float64 output keeps the double.
__device__ __forceinline__ void dev_dequant_store(void* out, int64_t index, uint32_t code, double scale, double zero,
                                                  int meta, int out_dt) {
  if (meta == kF64 && out_dt == kF64) {
    ((double*)out)[index] = __dadd_rn(__dmul_rn((double)code, scale), zero);
  } else {
    dev_store(out, index, dev_dequant(code, scale, zero, meta, out_dt), out_dt);
  }
}

__device__ __forceinline__ float dev_group_scale(float mn, float mx, float qmax, int dt) {
  float range = dev_round_to(__fsub_rn(mx, mn), dt);
  const float eps = quant_eps(dt);
  if (!(range >= eps)) range = eps;
  return dev_round_to(__fdiv_rn(range, qmax), dt);
}

__device__ __forceinline__ uint32_t dev_group_code(float x, float mn, float scale, float qmax, int dt) {
  const float diff = dev_round_to(__fsub_rn(x, mn), dt);
  float q = __builtin_rintf(dev_round_to(__fdiv_rn(diff, scale), dt));
  q = q < 0.0f ? 0.0f : q;
  q = q > qmax ? qmax : q;
  return (uint32_t)q;
}

// The same chain for float64 sources, in IEEE double (the reference keeps the
// source dtype, so a float64 tensor is quantized in float64; its eps is the
// double 1e-6, quantization.py:182-186, mixed.py:203-209).
__device__ __forceinline__ double dev_group_scale(double mn, double mx, double qmax, int) {
  double range = __dsub_rn(mx, mn);
  if (!(range >= 1.0e-6)) range = 1.0e-6;
  return __ddiv_rn(range, qmax);
}

__device__ __forceinline__ uint32_t dev_group_code(double x, double mn, double scale, double qmax, int) {
  double q = __builtin_rint(__ddiv_rn(__dsub_rn(x, mn), scale));
  q = q < 0.0 ? 0.0 : q;
  q = q > qmax ? qmax : q;
  return (uint32_t)q;
}

__device__ __forceinline__ float wave_max(float v) {
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

}  // namespace dkv
