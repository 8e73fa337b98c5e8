// Decode-step preparation for the Qwen3 fused attention adapter (gfx950, wave64).
//
// One launch replaces, for one new token per sequence, the adapter's query/key
// RMSNorm, the rotary embedding and the cache append of the new key/value
// (reference src/dart/integrations/qwen3.py:46-69, the Transformers Qwen3
// RMSNorm and apply_rotary_pos_emb it calls, and huggingface.py:68's append
// into the held tail).  The arithmetic follows those torch ops: RMSNorm in fp32
// (x * rsqrt(mean(x^2) + eps)), rounded to the cache dtype, times the weight
// (rounded); then q*cos and rotate_half(q)*sin each rounded and their sum
// rounded.  The mean is a wave reduction, so its fp32 summation order differs
// from torch's; results can differ from the eager ops by one unit in the last
// place of the cache dtype on rare elements.
//
// One wave per (sequence, head): heads [0, Hq) are query heads (normalized,
// rotated, written to q_out), [Hq, Hq + Hkv) key heads (normalized, rotated,
// written to the tail at the device position), [Hq + Hkv, Hq + 2 Hkv) value
// heads (copied to the tail).  Lane l holds channels l and l + 64, the pair
// rotate_half mixes.
#include <hip/hip_runtime.h>
#include <math.h>

#include "dkv_capi_util.h"
#include "dkv_device.h"

using namespace dkv;

namespace {

constexpr int kPrepDim = 128;

__device__ __forceinline__ float wave_sum64(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__global__ void __launch_bounds__(256) decode_prep(dkv_decode_prep_args a) {
  const int lane = threadIdx.x & 63;
  const int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int heads = (int)(a.Hq + 2 * a.Hkv);
  if (unit >= a.B * heads) return;
  const int b = (int)(unit / heads), h = (int)(unit % heads);
  const int dt = (int)a.dtype;
  const int64_t in = b * a.qkv_sb + (int64_t)h * kPrepDim;
  float x0 = dev_load(a.qkv, in + lane, dt);
  float x1 = dev_load(a.qkv, in + lane + 64, dt);
  const int64_t pos = *a.tail_pos;
  if (pos < 0 || pos >= a.cap) return;  // the caller keeps the position inside the tail
  if (h >= a.Hq + a.Hkv) {  // value head: copy into the tail
    const int kvh = h - (int)(a.Hq + a.Hkv);
    const int64_t out = ((b * a.Hkv + kvh) * a.cap + pos) * kPrepDim;
    dev_store(a.tail_value, out + lane, x0, dt);
    dev_store(a.tail_value, out + lane + 64, x1, dt);
    return;
  }
  const bool query = h < a.Hq;
  const void* w = query ? a.q_weight : a.k_weight;
  const float var = wave_sum64(x0 * x0 + x1 * x1) * (1.0f / kPrepDim);
  const float r = rsqrtf(var + (float)a.eps);
  const float n0 = dev_round_to(dev_round_to(x0 * r, dt) * dev_load(w, lane, dt), dt);
  const float n1 = dev_round_to(dev_round_to(x1 * r, dt) * dev_load(w, lane + 64, dt), dt);
  // rotate_half: channel l (< 64) takes -x[l + 64], channel l + 64 takes x[l]
  const float c0 = dev_load(a.cos, lane, dt), c1 = dev_load(a.cos, lane + 64, dt);
  const float s0 = dev_load(a.sin, lane, dt), s1 = dev_load(a.sin, lane + 64, dt);
  const float y0 = dev_round_to(dev_round_to(n0 * c0, dt) + dev_round_to(-n1 * s0, dt), dt);
  const float y1 = dev_round_to(dev_round_to(n1 * c1, dt) + dev_round_to(n0 * s1, dt), dt);
  if (query) {
    const int64_t out = (b * a.Hq + h) * kPrepDim;
    dev_store(a.q_out, out + lane, y0, dt);
    dev_store(a.q_out, out + lane + 64, y1, dt);
  } else {
    const int kvh = h - (int)a.Hq;
    const int64_t out = ((b * a.Hkv + kvh) * a.cap + pos) * kPrepDim;
    dev_store(a.tail_key, out + lane, y0, dt);
    dev_store(a.tail_key, out + lane + 64, y1, dt);
  }
}

}  // namespace

extern "C" int dkv_decode_prep(const dkv_decode_prep_args* args, void* stream) {
  DKV_CHECK(args != nullptr, DKV_ERR_INVALID, "dkv_decode_prep: args is NULL");
  const dkv_decode_prep_args& a = *args;
  DKV_CHECK(a.D == kPrepDim, DKV_ERR_UNSUPPORTED, "dkv_decode_prep: head_dim must be 128");
  DKV_CHECK(a.dtype == kBF16 || a.dtype == kF16, DKV_ERR_UNSUPPORTED, "dkv_decode_prep: bf16 or fp16 tensors only");
  DKV_CHECK(a.B > 0 && a.Hq > 0 && a.Hkv > 0 && a.Hq % a.Hkv == 0, DKV_ERR_INVALID,
            "dkv_decode_prep: bad head counts");
  DKV_CHECK(a.cap > 0, DKV_ERR_INVALID, "dkv_decode_prep: tail capacity must be positive");
  DKV_CHECK(a.qkv_sb >= (a.Hq + 2 * a.Hkv) * a.D, DKV_ERR_INVALID, "dkv_decode_prep: qkv row stride too small");
  DKV_CHECK(a.qkv && a.q_weight && a.k_weight && a.cos && a.sin && a.q_out && a.tail_key && a.tail_value &&
                a.tail_pos,
            DKV_ERR_INVALID, "dkv_decode_prep: NULL pointer");
  const int64_t units = a.B * (a.Hq + 2 * a.Hkv);
  hipLaunchKernelGGL(decode_prep, dim3((unsigned)((units + 3) / 4)), dim3(256), 0, (hipStream_t)stream, a);
  return dkv_check_launch("dkv_decode_prep");
}
