// The dense rest of a decode call (the sink and held-tail segments, one wave
// per 32-token chunk) and the merge of every split record of a (batch, kv
// head) pair: shared by the decode entry point's own kernels and by the page
// kernels, which can run the dense chunks in their own launch.
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "../../include/dartkv.h"
#include "dkv_device.h"

namespace dkv {

struct DecodeParams {
  dkv_decode_args a;
  int group;        // query heads per KV head
  int n_total;      // segments this kernel walks, including the tail
  int splits;       // splits of this kernel
  int split_offset; // first workspace split slot this kernel writes
  int split_stride; // split slots per (batch, query head) record
  int skip_first;   // descriptor entries [skip_first, skip_first + skip_count)
  int skip_count;   // belong to the fast page kernel
};

// Segment v of the general kernel's sequence: descriptor entries outside the
// fast range, then the tail.
__device__ __forceinline__ dkv_segment general_segment(const DecodeParams& p, int v) {
  const int rest = (int)p.a.n_segments - p.skip_count;
  if (v >= rest) {
    dkv_segment t = p.a.tail;
    if (p.a.tail_tokens_dev != nullptr) {
      const int64_t n = *p.a.tail_tokens_dev;
      t.tokens = (int32_t)(n < 0 ? 0 : (n < t.tokens ? n : t.tokens));
    }
    return t;
  }
  return p.a.segments[v < p.skip_first ? v : v + p.skip_count];
}

constexpr int kDenseWaves = 4;
constexpr int kDenseChunk = 32;
constexpr int kDenseDim = 128;
constexpr int kDenseMaxGroup = 8;        // the dense kernels of their own (decode.hip)
constexpr int kDenseFusedMaxGroup = 16;  // dense chunk waves inside the Dart page kernel's launch

// Every head slot of the dense kernel computes (the query of slots >= G is
// zero), so the unrolled loops carry no per-head branches; only the record
// writes are guarded.
#define DKV_ALL_HEADS(h) _Pragma("unroll") for (int h = 0; h < MG; ++h)
#define DKV_FOR_HEAD(h) _Pragma("unroll") for (int h = 0; h < MG; ++h) if (h < G)

template <bool BF>
__device__ __forceinline__ float dense_elem(uint16_t bits) {
  return BF ? bf16_to_f32(bits) : (float)__builtin_bit_cast(_Float16, bits);
}

// An offset the compiler must treat as computed from every dep[h]: reads
// addressed with it cannot be issued before all of them are.  (Depending on
// one head only let the compiler finish that head's chain first and keep the
// other heads' query values live across all steps.)
template <int MG>
__device__ __forceinline__ int after(int offset, const float (&dep)[MG]) {
#pragma unroll
  for (int h = 0; h < MG; ++h) asm volatile("" : "+v"(offset) : "v"(dep[h]));
  return offset;
}

// MG consecutive floats from LDS (one read for MG = 2, 4; two for 8)
template <int MG>
__device__ __forceinline__ void lds_heads(const float* src, float (&x)[MG]) {
  if (MG == 1) {
    x[0] = src[0];
  } else if (MG == 2) {
    const float2 v = *(const float2*)src;
    x[0] = v.x; x[1 % MG] = v.y;
  } else {
#pragma unroll
    for (int j = 0; j < MG; j += 4) {
      const float4 v = *(const float4*)(src + j);
      x[j] = v.x; x[(j + 1) % MG] = v.y; x[(j + 2) % MG] = v.z; x[(j + 3) % MG] = v.w;
    }
  }
}

// Chunk `chunk` of rest segment v of (batch, kv head) bhi, by one wave; qs
// and ws are the wave's LDS (kDenseDim * MG and kDenseChunk * MG floats).
template <int MG, bool BF>
__device__ __forceinline__ void dense_chunk(const DecodeParams& p, int chunks, int bhi, int v, int chunk, int lane,
                                            float* qs, float* ws) {
  const dkv_decode_args& a = p.a;
  const int b = bhi / (int)a.Hkv, kvh = bhi % (int)a.Hkv;
  const int64_t bh = (int64_t)bhi;
  const int G = p.group;

  const dkv_segment seg = general_segment(p, v);
  const bool ok = seg.key_kind == DKV_KEY_DENSE && seg.value_kind == DKV_VALUE_DENSE &&
                  seg.tokens <= chunks * kDenseChunk;
  const int t0 = chunk * kDenseChunk;
  const int nt = ok ? max(0, min(kDenseChunk, seg.tokens - t0)) : 0;
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(1))) const u32x4 gu4;
  typedef __attribute__((address_space(1))) const uint32_t gu32;
  const uint16_t* kbase = (const uint16_t*)(seg.key[0] + 2 * (uint64_t)(bh * seg.key_bh[0]));
  const uint16_t* vbase = (const uint16_t*)(seg.value[0] + 2 * (uint64_t)(bh * seg.value_bh[0]));
  const int kt = lane & (kDenseChunk - 1), khalf = lane >> 5;  // token, channel half of the Q K lane
  const int last = nt > 0 ? nt - 1 : 0;

  // K rows (8 x 16 B per lane) and V pairs (one dword per token), issued
  // before the query so one wait covers them; the query goes to LDS as fp32
  u32x4 krow[8];
  uint32_t vpair[kDenseChunk];
  if (nt > 0) {
    gu4* krp = (gu4*)(kbase + (int64_t)(t0 + (kt < nt ? kt : last)) * kDenseDim + 64 * khalf);
#pragma unroll
    for (int u = 0; u < 8; ++u) krow[u] = krp[u];
#pragma unroll
    for (int u = 0; u < kDenseChunk; ++u)
      vpair[u] = *(gu32*)(vbase + (int64_t)(t0 + (u < nt ? u : last)) * kDenseDim + 2 * lane);
  }
  {
    float qv[kDenseDim * MG / 64];
    dev_load_n(a.query, (int)a.q_dtype, qv, [&](int r) -> int64_t {
      const int i = lane + 64 * r, c = i / MG, h = i % MG;
      return h < G ? (int64_t)b * a.q_sb + (int64_t)(kvh * G + h) * a.q_sh + c : -1;
    });
#pragma unroll
    for (int r = 0; r < kDenseDim * MG / 64; ++r) qs[lane + 64 * r] = qv[r];
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  float m[MG], l[MG], pv0[MG], pv1[MG];
  if (nt > 0) {
    // ---- logits: 8 steps of 8 channels ----
    float logit[MG];
    DKV_ALL_HEADS(h) logit[h] = 0.f;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const uint32_t ww[4] = {krow[u].x, krow[u].y, krow[u].z, krow[u].w};
      const int qo = after<MG>((64 * khalf + 8 * u) * MG, logit);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float kv = dense_elem<BF>((uint16_t)(ww[i / 2] >> (16 * (i % 2))));
        float q[MG];
        lds_heads<MG>(qs + qo + i * MG, q);
        DKV_ALL_HEADS(h) logit[h] = fmaf(q[h], kv, logit[h]);
      }
    }
    const float scale = (float)a.scale;
    DKV_ALL_HEADS(h) {
      const float lg = kt < nt ? (logit[h] + __shfl_xor(logit[h], 32, 64)) * scale : -INFINITY;
      m[h] = wave_max(lg);
      const float w = kt < nt ? expf(lg - m[h]) : 0.f;
      if (khalf == 0) ws[kt * MG + h] = w;
      l[h] = wave_sum(w) * 0.5f;  // every weight appears in two lanes
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- weighted values: channels 2 lane, 2 lane + 1, 4 steps of 8 tokens ----
    DKV_ALL_HEADS(h) pv0[h] = pv1[h] = 0.f;
#pragma unroll
    for (int u0 = 0; u0 < kDenseChunk; u0 += 8) {
      const int wo = after<MG>(u0 * MG, pv1);
#pragma unroll
      for (int u = u0; u < u0 + 8; ++u) {
        const float v0 = dense_elem<BF>((uint16_t)vpair[u]);
        const float v1 = dense_elem<BF>((uint16_t)(vpair[u] >> 16));
        float w[MG];
        lds_heads<MG>(ws + wo + (u - u0) * MG, w);
        DKV_ALL_HEADS(h) {
          pv0[h] = fmaf(w[h], v0, pv0[h]);
          pv1[h] = fmaf(w[h], v1, pv1[h]);
        }
      }
    }
  } else {
    DKV_ALL_HEADS(h) {
      m[h] = -INFINITY;
      l[h] = pv0[h] = pv1[h] = 0.f;
    }
  }

  float* wsp = (float*)a.workspace;
  DKV_FOR_HEAD(h) {
    const int hq = kvh * G + h;
    float* rec =
        wsp + (((int64_t)b * a.Hq + hq) * p.split_stride + p.split_offset + (int64_t)v * chunks + chunk) * (kDenseDim + 2);
    if (lane == 0) {
      // a segment this kernel cannot read (a caller that passed no host copy of
      // the descriptors to check) poisons its record (NaN output)
      rec[0] = ok ? m[h] : NAN;
      rec[1] = l[h];
    }
    rec[2 + 2 * lane] = pv0[h];
    rec[3 + 2 * lane] = pv1[h];
  }
}

// Combine the split records of query heads kvh * G + h (h < G) of batch b with
// the log-sum-exp rule, then out = acc / max(sum, 1e-20) (attention.py:86).
// Same arithmetic and summation order for every thread count: per head, the
// maximum and the sum run over the splits in order; each output channel sums
// even and odd splits separately and adds the two.  wgt / lsum: G * S floats of
// LDS each; mx / den: G floats.  Threads tid = 0 .. nt - 1 take part; sync()
// orders their LDS traffic (a workgroup barrier, or a wave's).
template <class Sync>
__device__ __forceinline__ void merge_heads(const DecodeParams& p, int b, int hq0, int G, float* wgt, float* lsum,
                                            float* mx, float* den, int tid, int nt, Sync sync) {
  const dkv_decode_args& a = p.a;
  const int D = (int)a.D, S = p.split_stride;
  const float* ws = (const float*)a.workspace + ((int64_t)b * a.Hq + hq0) * S * (D + 2);
  for (int i = tid; i < G * S; i += nt) {
    wgt[i] = ws[(int64_t)i * (D + 2)];
    lsum[i] = ws[(int64_t)i * (D + 2) + 1];
  }
  sync();
  if (tid < G) {
    const float* w = wgt + tid * S;
    float M = -INFINITY;
    for (int s = 0; s < S; ++s) M = fmaxf(M, w[s]);
    mx[tid] = M;
  }
  sync();
  for (int i = tid; i < G * S; i += nt) {
    const float ms = wgt[i];
    wgt[i] = ms == -INFINITY ? 0.f : expf(ms - mx[i / S]);
  }
  sync();
  if (tid < G) {
    const float* w = wgt + tid * S;
    const float* l = lsum + tid * S;
    float L = 0.f;
    for (int s = 0; s < S; ++s) L += l[s] * w[s];
    den[tid] = fmaxf(L, 1e-20f);
  }
  sync();
  for (int i = tid; i < G * D; i += nt) {
    const int h = i / D, c = i % D;
    const float* w = wgt + h * S;
    const float* rec = ws + (int64_t)h * S * (D + 2) + 2 + c;
    float o0 = 0.f, o1 = 0.f;
    int s = 0;
    for (; s + 8 <= S; s += 8) {  // eight records' loads in flight, then the same sums in order
      float r[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) r[j] = rec[(int64_t)(s + j) * (D + 2)];
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        o0 += r[j] * w[s + j];
        o1 += r[j + 1] * w[s + j + 1];
      }
    }
    for (; s + 1 < S; s += 2) {
      o0 += rec[(int64_t)s * (D + 2)] * w[s];
      o1 += rec[(int64_t)(s + 1) * (D + 2)] * w[s + 1];
    }
    if (s < S) o0 += rec[(int64_t)s * (D + 2)] * w[s];
    const float o = (o0 + o1) / den[h];
    const int hq = hq0 + h;
    dev_store(a.out, (int64_t)b * a.out_sb + (int64_t)hq * a.out_sh + c, o, (int)a.q_dtype);
    if (a.out_f32) a.out_f32[((int64_t)b * a.Hq + hq) * D + c] = o;
  }
}

}  // namespace dkv
