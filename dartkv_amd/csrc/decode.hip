// Single-token GQA decode attention over packed DartKV segments (gfx950).
//
// Split-K over segments: workgroup (split, kv_head, batch) streams its
// contiguous range of segments, keeps an online-softmax state (max, sum,
// acc[D]) for each of the query heads that share the KV head, and writes the
// partial state to the workspace.  A merge pass combines the splits with the
// log-sum-exp rule and applies the reference's final normalisation
// `acc / max(sum, 1e-20)` (reference src/dart/attention.py:86,
// src/dart/fused_attention.py:742).
//
// K/V elements are dequantized with the reference's rounding chain
// (code*scale and +zero rounded in the metadata dtype, then the cache dtype),
// so the values attended to are exactly those the reference's streamed
// attention sees (attention.py:74-77).
#include <hip/hip_runtime.h>

#include <mutex>
#include <math.h>

#include "dkv_capi_util.h"
#include "dkv_decode.h"
#include "dkv_dense.h"
#include "dkv_device.h"

using namespace dkv;

namespace {

constexpr int kThreads = 256;
constexpr int kMaxGroup = 16;   // query heads per KV head
constexpr int kMaxDim = 512;    // head_dim
constexpr int kChanPerThread = kMaxDim / kThreads;

__device__ __forceinline__ float key_value(const dkv_segment& s, int64_t bh, int c, int t, int D, const int32_t* inv,
                                           int cache_dt, int meta) {
  if (s.key_kind == DKV_KEY_DENSE) {
    return dev_load((const void*)s.key[0], bh * s.key_bh[0] + (int64_t)t * D + c, cache_dt);
  }
  const int kg = s.key_group;
  const int G = (s.tokens + kg - 1) / kg;
  const int g = t / kg;
  uint32_t code;
  if (s.key_kind == DKV_KEY_UNIFORM) {
    const int per_byte = 8 / s.key_bits;
    const int pk = (G * kg + per_byte - 1) / per_byte;
    const uint8_t byte = ((const uint8_t*)s.key[0])[bh * s.key_bh[0] + (int64_t)c * pk + t / per_byte];
    code = (byte >> ((t % per_byte) * s.key_bits)) & ((1u << s.key_bits) - 1u);
  } else {
    const int nb = (kg + 3) / 4;
    const int w = t % kg;
    const uint8_t lo = ((const uint8_t*)s.key[0])[bh * s.key_bh[0] + ((int64_t)c * G + g) * nb + w / 4];
    code = (lo >> ((w % 4) * 2)) & 3u;
    const int slot = inv[c];
    if (slot >= 0) {
      const uint8_t hi = ((const uint8_t*)s.key[1])[bh * s.key_bh[1] + ((int64_t)slot * G + g) * nb + w / 4];
      code |= ((hi >> ((w % 4) * 2)) & 3u) << 2;
    }
  }
  const int64_t mi = (int64_t)c * G + g;
  return dev_dequant(code, dev_load_meta((const void*)s.key[3], bh * s.key_bh[3] + mi, meta),
                     dev_load_meta((const void*)s.key[4], bh * s.key_bh[4] + mi, meta), meta, cache_dt);
}

__device__ __forceinline__ float value_value(const dkv_segment& s, int64_t bh, int t, int c, int D, int cache_dt,
                                             int meta) {
  if (s.value_kind == DKV_VALUE_DENSE) {
    return dev_load((const void*)s.value[0], bh * s.value_bh[0] + (int64_t)t * D + c, cache_dt);
  }
  const int vg = s.value_group;
  const int Gv = (D + vg - 1) / vg;
  const int per_byte = 8 / s.value_bits;
  const int pv = (Gv * vg + per_byte - 1) / per_byte;
  const uint8_t byte = ((const uint8_t*)s.value[0])[bh * s.value_bh[0] + (int64_t)t * pv + c / per_byte];
  const uint32_t code = (byte >> ((c % per_byte) * s.value_bits)) & ((1u << s.value_bits) - 1u);
  const int64_t mi = (int64_t)t * Gv + c / vg;
  return dev_dequant(code, dev_load_meta((const void*)s.value[1], bh * s.value_bh[1] + mi, meta),
                     dev_load_meta((const void*)s.value[2], bh * s.value_bh[2] + mi, meta), meta, cache_dt);
}

// MG is a compile-time bound on the query heads per KV head, so the per-head
// state below stays in registers: DKV_FOR_HEAD unrolls over MG heads and skips
// heads >= G.
#define DKV_FOR_HEAD(h) _Pragma("unroll") for (int h = 0; h < MG; ++h) if (h < G)
template <int MG>
__global__ void __launch_bounds__(kThreads) decode_split_general(DecodeParams p) {
  const dkv_decode_args& a = p.a;
  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int D = (int)a.D, G = p.group, Hq = (int)a.Hq;
  const int cache_dt = (int)a.cache_dtype, meta = (int)a.meta_dtype;
  const int64_t bh = (int64_t)b * a.Hkv + kvh;
  const float scale = (float)a.scale;

  __shared__ float q_s[kMaxGroup * kMaxDim];
  __shared__ float w_s[kMaxGroup * kThreads];
  __shared__ float red_s[kMaxGroup * (kThreads / 64)];
  __shared__ int32_t inv_s[kMaxDim];

  for (int i = threadIdx.x; i < G * D; i += kThreads) {
    const int h = i / D, c = i % D;
    q_s[i] = dev_load(a.query, (int64_t)b * a.q_sb + (int64_t)(kvh * G + h) * a.q_sh + c, (int)a.q_dtype);
  }

  float m[MG], l[MG], acc[MG][kChanPerThread];
#pragma unroll
  for (int h = 0; h < MG; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
    for (int j = 0; j < kChanPerThread; ++j) acc[h][j] = 0.f;
  }

  const int s0 = (int)(((int64_t)split * p.n_total) / p.splits);
  const int s1 = (int)(((int64_t)(split + 1) * p.n_total) / p.splits);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;

  for (int si = s0; si < s1; ++si) {
    const dkv_segment seg = general_segment(p, si);
    __syncthreads();
    if (seg.key_kind == DKV_KEY_MIXED) {
      for (int c = threadIdx.x; c < D; c += kThreads) inv_s[c] = -1;
      __syncthreads();
      const int32_t* idx = (const int32_t*)seg.key[2] + bh * seg.key_bh[2];
      for (int j = threadIdx.x; j < seg.promoted; j += kThreads) {
        const int32_t ch = idx[j];
        if (ch >= 0 && ch < D) inv_s[ch] = j;
      }
    }
    __syncthreads();
    const bool dense16 = seg.key_kind == DKV_KEY_DENSE && (cache_dt == kBF16 || cache_dt == kF16) && (D % 8) == 0 &&
                         (seg.key[0] % 16) == 0 && ((seg.key_bh[0] * 2) % 16) == 0;
    for (int t0 = 0; t0 < seg.tokens; t0 += kThreads) {
      const int nt = min(kThreads, seg.tokens - t0);
      // ---- logits for this tile: thread = token ----
      float logit[MG];
      DKV_FOR_HEAD(h) logit[h] = 0.f;
      if ((int)threadIdx.x < nt) {
        const int t = t0 + threadIdx.x;
        if (dense16) {
          // dense 16-bit keys: 16-byte loads, 4 in flight, same channel order
          const uint4* row = (const uint4*)((const uint16_t*)seg.key[0] + bh * seg.key_bh[0] + (int64_t)t * D);
          for (int c0 = 0; c0 < D; c0 += 32) {
            uint4 w4[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) w4[u] = (c0 + 8 * u < D) ? row[c0 / 8 + u] : make_uint4(0, 0, 0, 0);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              if (c0 + 8 * u >= D) break;
              const uint32_t ww[4] = {w4[u].x, w4[u].y, w4[u].z, w4[u].w};
#pragma unroll
              for (int i = 0; i < 8; ++i) {
                const uint16_t bits = (uint16_t)(ww[i / 2] >> (16 * (i % 2)));
                const float kv = cache_dt == kBF16 ? bf16_to_f32(bits) : (float)__builtin_bit_cast(_Float16, bits);
                const int c = c0 + 8 * u + i;
                DKV_FOR_HEAD(h) logit[h] = fmaf(q_s[h * D + c], kv, logit[h]);
              }
            }
          }
        } else {
          for (int c = 0; c < D; ++c) {
            const float kv = key_value(seg, bh, c, t, D, inv_s, cache_dt, meta);
            DKV_FOR_HEAD(h) logit[h] = fmaf(q_s[h * D + c], kv, logit[h]);
          }
        }
        DKV_FOR_HEAD(h) logit[h] = logit[h] * scale;
      } else {
        DKV_FOR_HEAD(h) logit[h] = -INFINITY;
      }
      // ---- tile max per head ----
      DKV_FOR_HEAD(h) {
        const float wm = wave_max(logit[h]);
        if (lane == 0) red_s[h * (kThreads / 64) + wave] = wm;
      }
      __syncthreads();
      float new_m[MG], old_w[MG];
      DKV_FOR_HEAD(h) {
        float tm = red_s[h * (kThreads / 64)];
        for (int w = 1; w < kThreads / 64; ++w) tm = fmaxf(tm, red_s[h * (kThreads / 64) + w]);
        new_m[h] = fmaxf(m[h], tm);
        old_w[h] = expf(m[h] - new_m[h]);
      }
      __syncthreads();
      DKV_FOR_HEAD(h) {
        const float w = (int)threadIdx.x < nt ? expf(logit[h] - new_m[h]) : 0.f;
        w_s[h * kThreads + threadIdx.x] = w;
        const float ws = wave_sum(w);
        if (lane == 0) red_s[h * (kThreads / 64) + wave] = ws;
      }
      __syncthreads();
      DKV_FOR_HEAD(h) {
        float ts = 0.f;
        for (int w = 0; w < kThreads / 64; ++w) ts += red_s[h * (kThreads / 64) + w];
        l[h] = l[h] * old_w[h] + ts;
        m[h] = new_m[h];
      }
      // ---- weighted values: thread = channel ----
      for (int j = 0; j < kChanPerThread; ++j) {
        const int c = threadIdx.x + j * kThreads;
        if (c >= D) break;
        float pv[MG];
        DKV_FOR_HEAD(h) pv[h] = 0.f;
        if (seg.value_kind == DKV_VALUE_DENSE && (cache_dt == kBF16 || cache_dt == kF16)) {
          // dense 16-bit values: 8 loads in flight per thread, coalesced across channels
          const uint16_t* vcol = (const uint16_t*)seg.value[0] + bh * seg.value_bh[0] + (int64_t)t0 * D + c;
          int t = 0;
          for (; t + 8 <= nt; t += 8) {
            uint16_t vb[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) vb[i] = vcol[(int64_t)(t + i) * D];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              const float vv = cache_dt == kBF16 ? bf16_to_f32(vb[i]) : (float)__builtin_bit_cast(_Float16, vb[i]);
              DKV_FOR_HEAD(h) pv[h] = fmaf(w_s[h * kThreads + t + i], vv, pv[h]);
            }
          }
          for (; t < nt; ++t) {
            const uint16_t vb = vcol[(int64_t)t * D];
            const float vv = cache_dt == kBF16 ? bf16_to_f32(vb) : (float)__builtin_bit_cast(_Float16, vb);
            DKV_FOR_HEAD(h) pv[h] = fmaf(w_s[h * kThreads + t], vv, pv[h]);
          }
        } else {
          for (int t = 0; t < nt; ++t) {
            const float vv = value_value(seg, bh, t0 + t, c, D, cache_dt, meta);
            DKV_FOR_HEAD(h) pv[h] = fmaf(w_s[h * kThreads + t], vv, pv[h]);
          }
        }
        DKV_FOR_HEAD(h) acc[h][j] = acc[h][j] * old_w[h] + pv[h];
      }
      __syncthreads();
    }
  }

  // ---- partial state: ws[(b, hq, split)] = {max, sum, acc[D]} ----
  float* ws = (float*)a.workspace;
  DKV_FOR_HEAD(h) {
    const int hq = kvh * G + h;
    float* rec = ws + (((int64_t)b * Hq + hq) * p.split_stride + p.split_offset + split) * (D + 2);
    if (threadIdx.x == 0) {
      rec[0] = m[h];
      rec[1] = l[h];
    }
    for (int j = 0; j < kChanPerThread; ++j) {
      const int c = threadIdx.x + j * kThreads;
      if (c < D) rec[2 + c] = acc[h][j];
    }
  }
}

// Dense 16-bit segments (the sink and the held tail): one wave per (batch,
// kv head, segment, 32-token chunk), fp32 dot products as the reference's
// eager attention computes them.  Q K: lane = (token, half of the channels),
// the two halves combined across lanes l and l^32; P V: lane = channel pair.
// The K and V rows are loaded straight into registers (rows past the chunk's
// tokens re-read its last row; their logits become -inf and their weights 0),
// the query and the softmax weights are read from LDS as broadcasts.  Each
// step's LDS reads are addressed through the previous step's accumulator, so
// only one step's values are live: unrolled whole, the compiler issued all
// 128 x MG query reads first and kept them in registers (one wave per SIMD).
// The wave
// writes one record at split slot split_offset + segment * chunks + chunk.
template <int MG, bool BF>
__global__ void __launch_bounds__(64 * kDenseWaves) decode_dense_rest(DecodeParams p, int chunks) {
  __shared__ __attribute__((aligned(16))) float qsh[kDenseWaves][kDenseDim * MG];    // [c][MG]
  __shared__ __attribute__((aligned(16))) float wsh[kDenseWaves][kDenseChunk * MG];  // [t][MG] weights
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int worker = blockIdx.x * kDenseWaves + wave;
  const int per_bh = p.n_total * chunks;
  if (worker >= (int)(p.a.B * p.a.Hkv) * per_bh) return;
  dense_chunk<MG, BF>(p, chunks, worker / per_bh, (worker % per_bh) / chunks, worker % chunks, lane, qsh[wave],
                      wsh[wave]);
}

// The dense rest segments and the merge in one launch: one block per (batch,
// kv head).  Its waves take the (segment, chunk) tasks of that pair in turn
// and write their records; after a barrier the block merges every record of
// the pair's query heads (the page kernel's were written by the launch
// before).  Saves the merge launch and its wait.  Up to 4 heads per KV head it
// keeps to 128 VGPRs, so two blocks share a CU.
constexpr int kDenseMergeWaves = 8;

template <int MG, bool BF>
__global__ void __launch_bounds__(64 * kDenseMergeWaves, MG <= 4 ? 4 : 2) decode_dense_merge(DecodeParams p, int chunks) {
  __shared__ __attribute__((aligned(16))) float qsh[kDenseMergeWaves][kDenseDim * MG];
  __shared__ __attribute__((aligned(16))) float wsh[kDenseMergeWaves][kDenseChunk * MG];
  __shared__ float mx[kDenseMaxGroup], den[kDenseMaxGroup];
  extern __shared__ float dyn[];  // [G][S] weights, [G][S] sums
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int bhi = blockIdx.x;
  const int tasks = p.n_total * chunks;
  for (int t = wave; t < tasks; t += kDenseMergeWaves)
    dense_chunk<MG, BF>(p, chunks, bhi, t / chunks, t % chunks, lane, qsh[wave], wsh[wave]);
  __syncthreads();
  const int G = p.group, S = p.split_stride;
  const int b = bhi / (int)p.a.Hkv, kvh = bhi % (int)p.a.Hkv;
  merge_heads(p, b, kvh * G, G, dyn, dyn + G * S, mx, den, (int)threadIdx.x, (int)blockDim.x,
              [] __device__() { __syncthreads(); });
}

// One block per (batch, query head): the merge alone.  With at most
// kMergeRegSplits records per query head, each channel's thread issues the
// loads of all its records before the weights are known, and wave 0 forms the
// weights (a wave maximum, then the split sums added in split order), so the
// kernel waits on one round of loads instead of two; every sum runs in
// merge_heads' order, so the results are the same bits.
constexpr int kMergeRegSplits = 32;

__global__ void __launch_bounds__(kThreads) decode_merge(DecodeParams p) {
  extern __shared__ float wsh[];  // [S] weights, [S] sums
  __shared__ float mx[1], den[1];
  const int bq = blockIdx.x;  // b * Hq + hq
  const dkv_decode_args& a = p.a;
  const int S = p.split_stride, D = (int)a.D, tid = (int)threadIdx.x;
  if (S > kMergeRegSplits || D > kThreads) {
    merge_heads(p, bq / (int)a.Hq, bq % (int)a.Hq, 1, wsh, wsh + S, mx, den, tid, (int)blockDim.x,
                [] __device__() { __syncthreads(); });
    return;
  }
  const float* ws = (const float*)a.workspace + (int64_t)bq * S * (D + 2);
  float r[kMergeRegSplits];
  if (tid < D) {
#pragma unroll
    for (int s = 0; s < kMergeRegSplits; ++s) r[s] = s < S ? ws[(int64_t)s * (D + 2) + 2 + tid] : 0.f;
  }
  if (tid < 64) {
    const float m = tid < S ? ws[(int64_t)tid * (D + 2)] : -INFINITY;
    const float l = tid < S ? ws[(int64_t)tid * (D + 2) + 1] : 0.f;
    float M = m;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
    const float w = m == -INFINITY ? 0.f : expf(m - M);
    if (tid < S) wsh[tid] = w;
    const float lw = l * w;
    float L = 0.f;
    for (int s = 0; s < S; ++s) L += __shfl(lw, s, 64);
    if (tid == 0) den[0] = fmaxf(L, 1e-20f);
  }
  __syncthreads();
  if (tid < D) {
    float o0 = 0.f, o1 = 0.f;
#pragma unroll
    for (int s = 0; s < kMergeRegSplits; s += 2) {
      if (s < S) o0 += r[s] * wsh[s];
      if (s + 1 < S) o1 += r[s + 1] * wsh[s + 1];
    }
    const float o = (o0 + o1) / den[0];
    const int b = bq / (int)a.Hq, hq = bq % (int)a.Hq;
    dev_store(a.out, (int64_t)b * a.out_sb + (int64_t)hq * a.out_sh + tid, o, (int)a.q_dtype);
    if (a.out_f32) a.out_f32[(int64_t)bq * D + tid] = o;
  }
}

}  // namespace

// Record a caller's timing event (if any) on the stream.
static int record_event(void* ev, hipStream_t s) {
  if (ev == nullptr) return DKV_OK;
  const hipError_t e = hipEventRecord((hipEvent_t)ev, s);
  DKV_CHECK(e == hipSuccess, DKV_ERR_HIP, "dkv_decode_attention: hipEventRecord failed: %s", hipGetErrorString(e));
  return DKV_OK;
}

// ---------------------------------------------------------------------------
// Static scratch for dkv_decode_attention_noalloc: the split records live in a
// file-scope device array instead of a caller workspace.  Every GPU the
// library runs on holds its own copy until the process ends.  In host code
// `scratch` only names the array; its device address on the current GPU comes
// from hipGetSymbolAddress, fetched once per device and kept in
// g_scratch_ptr.
// ---------------------------------------------------------------------------
namespace {
constexpr int64_t kScratchBytes = (int64_t)32 << 20;
constexpr int kScratchMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
std::mutex g_scratch_mu;
void* g_scratch_ptr[kScratchMaxDevices] = {};

// Device address of `scratch` on the current device (looked up on the first
// call per device, with that device current).
int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  DKV_CHECK(e == hipSuccess, DKV_ERR_HIP, "dkv_decode_attention_noalloc: hipGetDevice failed: %s",
            hipGetErrorString(e));
  DKV_CHECK(dev >= 0 && dev < kScratchMaxDevices, DKV_ERR_UNSUPPORTED,
            "dkv_decode_attention_noalloc: device %d is beyond the %d devices it supports", dev, kScratchMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    DKV_CHECK(e == hipSuccess && ptr != nullptr, DKV_ERR_HIP,
              "dkv_decode_attention_noalloc: hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return DKV_OK;
}
}  // namespace

static bool float_dtype(int64_t dt) { return dt == dkv::kF32 || dt == dkv::kF16 || dt == dkv::kBF16 || dt == dkv::kF64; }

extern "C" int64_t dkv_decode_scratch_bytes(void) { return kScratchBytes; }

extern "C" int dkv_decode_attention_noalloc(const dkv_decode_args* args, void* stream) {
  DKV_CHECK(args != nullptr, DKV_ERR_INVALID, "args is NULL");
  dkv_decode_args a = *args;
  const bool fast = a.fast_count > 0;
  const int64_t rest = a.n_segments - (fast ? a.fast_count : 0) + (a.tail.tokens > 0 ? 1 : 0);
  const int64_t splits = (fast ? a.fast_splits : 0) + (rest > 0 ? a.n_splits : 0);
  const int64_t need = dkv_decode_workspace_bytes(a.B, a.Hq, a.D, splits);
  DKV_CHECK(need <= kScratchBytes, DKV_ERR_INVALID,
            "dkv_decode_attention_noalloc: the split records need %lld bytes, more than the %lld bytes of static "
            "scratch; use fewer splits or dkv_decode_attention with a workspace",
            (long long)need, (long long)kScratchBytes);
  void* ptr = nullptr;
  const int rc = scratch_address(&ptr);
  if (rc != DKV_OK) return rc;
  a.workspace = ptr;
  a.workspace_bytes = kScratchBytes;
  return dkv_decode_attention(&a, stream);
}

extern "C" int64_t dkv_decode_workspace_bytes(int64_t B, int64_t Hq, int64_t D, int64_t n_splits) {
  return B * Hq * n_splits * (D + 2) * (int64_t)sizeof(float);
}

// The caller's guarantees for the page kernels' run and for the dense rest
// (declared with dkv_decode_args), checked on the host: against
// segments_host when the caller passes one, and always for the tail.
static bool aligned16(uint64_t addr, int64_t bh, int elem_bytes) {
  return addr % 16 == 0 && (bh * elem_bytes) % 16 == 0;
}

static bool fast_page_ok(const dkv_decode_args& a, const dkv_segment& g) {
  if (!(g.tokens == 128 && g.key_group == 128 && g.value_kind == DKV_VALUE_UNIFORM &&
        g.value_group == a.fast_value_group))
    return false;
  if (a.fast_promoted > 0) {
    if (!(g.key_kind == DKV_KEY_MIXED && g.promoted == a.fast_promoted && g.value_bits == 2)) return false;
    if (!(aligned16(g.key[1], g.key_bh[1], 1) && aligned16(g.key[2], g.key_bh[2], 4))) return false;
  } else if (!(g.key_kind == DKV_KEY_UNIFORM && g.key_bits == a.fast_key_bits && g.value_bits == a.fast_value_bits)) {
    return false;
  }
  return aligned16(g.key[0], g.key_bh[0], 1) && aligned16(g.key[3], g.key_bh[3], 2) &&
         aligned16(g.key[4], g.key_bh[4], 2) && aligned16(g.value[0], g.value_bh[0], 1) &&
         aligned16(g.value[1], g.value_bh[1], 2) && aligned16(g.value[2], g.value_bh[2], 2);
}

static bool dense_rest_ok(const dkv_decode_args& a, const dkv_segment& g) {
  return g.key_kind == DKV_KEY_DENSE && g.value_kind == DKV_VALUE_DENSE && g.tokens <= a.rest_dense_tokens &&
         aligned16(g.key[0], g.key_bh[0], 2) && aligned16(g.value[0], g.value_bh[0], 2);
}

// The page kernels' grid (4 waves per workgroup) holds the page and the
// dense workers of a launch that merges.
static bool B_Hkv_rest_chunks_ok(const dkv_decode_args& a, int64_t rest, int64_t chunks) {
  return a.B * a.Hkv * (a.fast_splits + rest * chunks) < (int64_t)1 << 31;
}

static int check_segments(const dkv_decode_args& a, int64_t fast_count, bool dense_rest) {
  if (dense_rest && a.tail.tokens > 0)
    DKV_CHECK(dense_rest_ok(a, a.tail), DKV_ERR_INVALID,
              "rest_dense_tokens: the tail must be a dense bf16/fp16 segment of at most %lld tokens with 16-byte "
              "aligned rows", (long long)a.rest_dense_tokens);
  if (a.segments_host == nullptr) return DKV_OK;
  for (int64_t i = 0; i < a.n_segments; ++i) {
    const dkv_segment& g = a.segments_host[i];
    if (fast_count > 0 && i >= a.fast_first && i < a.fast_first + fast_count) {
      DKV_CHECK(fast_page_ok(a, g), DKV_ERR_INVALID, "descriptor %lld is not a page the fast page kernel reads",
                (long long)i);
    } else if (dense_rest) {
      DKV_CHECK(dense_rest_ok(a, g), DKV_ERR_INVALID,
                "rest_dense_tokens: descriptor %lld is not a dense segment of at most %lld tokens with 16-byte "
                "aligned rows", (long long)i, (long long)a.rest_dense_tokens);
    }
  }
  return DKV_OK;
}

extern "C" int dkv_decode_attention(const dkv_decode_args* args, void* stream) {
  DKV_CHECK(args != nullptr, DKV_ERR_INVALID, "args is NULL");
  dkv_decode_args a = *args;
  DKV_CHECK(a.B > 0 && a.Hq > 0 && a.Hkv > 0 && a.D > 0, DKV_ERR_INVALID, "bad decode shape");
  DKV_CHECK(a.Hq % a.Hkv == 0, DKV_ERR_INVALID, "query heads must be divisible by cache KV heads");
  DKV_CHECK(a.Hq / a.Hkv <= kMaxGroup, DKV_ERR_UNSUPPORTED, "at most %d query heads per KV head", kMaxGroup);
  DKV_CHECK(a.D <= kMaxDim, DKV_ERR_UNSUPPORTED, "head_dim %lld > %d", (long long)a.D, kMaxDim);
  DKV_CHECK(a.n_segments >= 0 && (a.n_segments == 0 || a.segments != nullptr), DKV_ERR_INVALID, "segments missing");
  DKV_CHECK(a.n_segments + (a.tail.tokens > 0 ? 1 : 0) > 0, DKV_ERR_INVALID, "cache is empty");
  DKV_CHECK(a.B <= 65535 && a.Hkv <= 65535, DKV_ERR_UNSUPPORTED, "batch or KV heads too large");
  DKV_CHECK(float_dtype(a.q_dtype) && float_dtype(a.cache_dtype) && float_dtype(a.meta_dtype), DKV_ERR_DTYPE,
            "query, cache and metadata dtypes must be f64, f32, f16 or bf16");
  const int64_t fast_count = a.fast_count;
  if (fast_count > 0) {
    DKV_CHECK(a.fast_first >= 0 && a.fast_first + fast_count <= a.n_segments, DKV_ERR_INVALID,
              "fast page range outside the descriptor table");
    DKV_CHECK(a.D == 128, DKV_ERR_UNSUPPORTED, "fast page path needs head_dim 128");
    const int64_t gq = a.Hq / a.Hkv;
    DKV_CHECK(gq == 1 || gq == 2 || gq == 4 || gq == 8 || (gq == 16 && a.fast_promoted > 0), DKV_ERR_UNSUPPORTED,
              "fast page path needs 1, 2, 4 or 8 query rows per KV head (16 on Dart pages)");
    DKV_CHECK(a.cache_dtype == dkv::kBF16 || a.cache_dtype == dkv::kF16, DKV_ERR_UNSUPPORTED,
              "fast page path needs a bf16 or fp16 cache");
    DKV_CHECK(a.meta_dtype == dkv::kF16, DKV_ERR_UNSUPPORTED, "fast page path needs fp16 metadata");
    DKV_CHECK(a.fast_value_group % 16 == 0 && a.fast_value_group > 0 && 128 % a.fast_value_group == 0,
              DKV_ERR_UNSUPPORTED, "fast page path needs a value group that is a multiple of 16 dividing 128");
    if (a.fast_promoted > 0) {
      DKV_CHECK(a.fast_promoted % 16 == 0 && a.fast_promoted >= 16 && a.fast_promoted <= 64, DKV_ERR_UNSUPPORTED,
                "fast page path needs 16, 32, 48 or 64 promoted channels");
      DKV_CHECK(a.fast_key_bits == 0 || a.fast_key_bits == 2, DKV_ERR_UNSUPPORTED,
                "fast page path: Dart pages have 2-bit base key codes");
      DKV_CHECK(a.fast_value_bits == 0 || a.fast_value_bits == 2, DKV_ERR_UNSUPPORTED,
                "fast page path: Dart pages need 2-bit values");
      DKV_CHECK(a.fast_splits >= 1 && a.fast_splits <= fast_count, DKV_ERR_INVALID, "fast_splits out of range");
      DKV_CHECK(dkv::fast_decode_max_loads((int)a.fast_promoted, (int)(128 / a.fast_value_group)) < 16,
                DKV_ERR_UNSUPPORTED, "fast page path: value group too small");
    } else {
      DKV_CHECK((a.fast_key_bits == 2 || a.fast_key_bits == 4 || a.fast_key_bits == 8) &&
                    (a.fast_value_bits == 2 || a.fast_value_bits == 4 || a.fast_value_bits == 8),
                DKV_ERR_UNSUPPORTED, "fast uniform pages need 2, 4 or 8-bit keys and values");
      DKV_CHECK(a.fast_splits >= 1 && a.fast_splits <= 2 * fast_count, DKV_ERR_INVALID, "fast_splits out of range");
      DKV_CHECK(dkv::uniform_decode_max_loads((int)a.fast_key_bits, (int)a.fast_value_bits,
                                              (int)(128 / a.fast_value_group)) < 16,
                DKV_ERR_UNSUPPORTED, "fast uniform pages: too many loads in flight");
    }
  }
  const int64_t rest = a.n_segments - (fast_count > 0 ? fast_count : 0) + (a.tail.tokens > 0 ? 1 : 0);
  const int64_t general_splits = rest > 0 ? a.n_splits : 0;
  DKV_CHECK(rest == 0 || (a.n_splits >= 1 && a.n_splits <= 65535), DKV_ERR_INVALID, "n_splits out of range");
  const int64_t fast_splits = fast_count > 0 ? a.fast_splits : 0;
  const int64_t stride = fast_splits + general_splits;
  DKV_CHECK(stride <= 8192, DKV_ERR_UNSUPPORTED, "too many splits");
  DKV_CHECK(a.workspace_bytes >= dkv_decode_workspace_bytes(a.B, a.Hq, a.D, stride), DKV_ERR_INVALID,
            "workspace too small");
  {
    const int rc = check_segments(a, fast_count, rest > 0 && a.rest_dense_tokens > 0);
    if (rc != DKV_OK) return rc;
  }
  hipStream_t s = (hipStream_t)stream;
  DecodeParams p;
  p.a = a;
  p.group = (int)(a.Hq / a.Hkv);
  p.n_total = (int)rest;
  p.splits = (int)general_splits;
  p.split_offset = (int)fast_splits;
  p.split_stride = (int)stride;
  p.skip_first = fast_count > 0 ? (int)a.fast_first : 0;
  p.skip_count = fast_count > 0 ? (int)fast_count : 0;
  const bool dense_rest = rest > 0 && a.rest_dense_tokens > 0;
  const int64_t chunks = dense_rest ? (a.rest_dense_tokens + kDenseChunk - 1) / kDenseChunk : 0;
  if (dense_rest) {
    DKV_CHECK(a.n_splits == rest * chunks, DKV_ERR_INVALID,
              "rest_dense_tokens needs n_splits == non-page segments * ceil(rest_dense_tokens / %d)", kDenseChunk);
    DKV_CHECK(a.cache_dtype == dkv::kBF16 || a.cache_dtype == dkv::kF16, DKV_ERR_UNSUPPORTED,
              "rest_dense_tokens needs a bf16 or fp16 cache");
    // up to kDenseMaxGroup heads per KV head in the dense kernels of their own; 16 only as waves of the
    // Dart page kernel's launch
    const int max_group = fast_count > 0 && a.fast_promoted > 0 ? kDenseFusedMaxGroup : kDenseMaxGroup;
    DKV_CHECK(a.D == kDenseDim && p.group <= max_group, DKV_ERR_UNSUPPORTED,
              "rest_dense_tokens needs head_dim %d and at most %d query heads per KV head", kDenseDim, max_group);
  }
  if (fast_count > 0) {
    // With a dense rest, the page kernel's launch also runs the dense chunks
    // (extra waves beside the page waves, so their latency hides behind the
    // pages), and one merge launch follows.  Merging in the page launch itself
    // (the last wave of a pair merges, found with a device-scope counter) was
    // measured twice as slow: on this multi-XCD part every wave's device-scope
    // release writes back its L2.
    const bool fuse = dense_rest && B_Hkv_rest_chunks_ok(a, rest, chunks) &&
                      (size_t)2 * stride * sizeof(float) <= 64 * 1024;
    DKV_CHECK(!dense_rest || fuse || p.group <= kDenseMaxGroup, DKV_ERR_UNSUPPORTED,
              "rest_dense_tokens with more than %d query heads per KV head needs the dense chunks in the page "
              "kernel's launch (too many splits)", kDenseMaxGroup);
    dkv::FusedRest fr{&p, (int)chunks};
    int rc = record_event(a.fast_events[0], s);
    if (rc) return rc;
    rc = a.fast_promoted > 0
             ? dkv::launch_fast_decode(a, (int)a.fast_first, (int)fast_count, (int)a.fast_promoted,
                                       (int)a.fast_value_group, (int)fast_splits, (int)stride, s,
                                       fuse ? &fr : nullptr)
             : dkv::launch_uniform_decode(a, (int)a.fast_first, (int)fast_count, (int)a.fast_key_bits,
                                          (int)a.fast_value_bits, (int)a.fast_value_group, (int)fast_splits,
                                          (int)stride, s, fuse ? &fr : nullptr);
    if (rc) return rc;
    rc = record_event(a.fast_events[1], s);
    if (rc) return rc;
    if (fuse) {
      hipLaunchKernelGGL(decode_merge, dim3((unsigned)(a.B * a.Hq)), dim3(kThreads), 2 * stride * sizeof(float), s, p);
      return dkv_check_launch("dkv_decode_attention(merge)");
    }
  }
  if (dense_rest) {
    const int mg = p.group <= 1 ? 1 : p.group <= 2 ? 2 : p.group <= 4 ? 4 : 8;
    const size_t merge_lds = (size_t)2 * p.group * stride * sizeof(float);
    if (merge_lds <= 64 * 1024) {
      // dense chunks and the merge in one launch, one block per (batch, kv head)
      const dim3 grid((unsigned)(a.B * a.Hkv)), block(64 * kDenseMergeWaves);
      const int ch = (int)chunks;
#define DKV_DM_LAUNCH(MGV)                                                                                    \
  do {                                                                                                        \
    if (a.cache_dtype == dkv::kBF16)                                                                          \
      hipLaunchKernelGGL((decode_dense_merge<MGV, true>), grid, block, merge_lds, s, p, ch);                 \
    else hipLaunchKernelGGL((decode_dense_merge<MGV, false>), grid, block, merge_lds, s, p, ch);             \
  } while (0)
      if (mg == 1) DKV_DM_LAUNCH(1);
      else if (mg == 2) DKV_DM_LAUNCH(2);
      else if (mg == 4) DKV_DM_LAUNCH(4);
      else DKV_DM_LAUNCH(8);
#undef DKV_DM_LAUNCH
      return dkv_check_launch("dkv_decode_attention(dense + merge)");
    }
    const int64_t workers = a.B * a.Hkv * rest * chunks;
    const dim3 grid((unsigned)((workers + kDenseWaves - 1) / kDenseWaves)), block(64 * kDenseWaves);
    const int ch = (int)chunks;
#define DKV_DENSE_LAUNCH(MGV)                                                                  \
  do {                                                                                         \
    if (a.cache_dtype == dkv::kBF16) hipLaunchKernelGGL((decode_dense_rest<MGV, true>), grid, block, 0, s, p, ch); \
    else hipLaunchKernelGGL((decode_dense_rest<MGV, false>), grid, block, 0, s, p, ch);      \
  } while (0)
    if (mg == 1) DKV_DENSE_LAUNCH(1);
    else if (mg == 2) DKV_DENSE_LAUNCH(2);
    else if (mg == 4) DKV_DENSE_LAUNCH(4);
    else DKV_DENSE_LAUNCH(8);
#undef DKV_DENSE_LAUNCH
    int rc = dkv_check_launch("dkv_decode_attention(dense)");
    if (rc) return rc;
  } else if (general_splits > 0) {
    const dim3 grid((unsigned)general_splits, (unsigned)a.Hkv, (unsigned)a.B);
    if (p.group <= 1) hipLaunchKernelGGL(decode_split_general<1>, grid, dim3(kThreads), 0, s, p);
    else if (p.group <= 2) hipLaunchKernelGGL(decode_split_general<2>, grid, dim3(kThreads), 0, s, p);
    else if (p.group <= 4) hipLaunchKernelGGL(decode_split_general<4>, grid, dim3(kThreads), 0, s, p);
    else if (p.group <= 8) hipLaunchKernelGGL(decode_split_general<8>, grid, dim3(kThreads), 0, s, p);
    else hipLaunchKernelGGL(decode_split_general<16>, grid, dim3(kThreads), 0, s, p);
    int rc = dkv_check_launch("dkv_decode_attention(split)");
    if (rc) return rc;
  }
  const int merge_threads = (int)(a.D < 64 ? 64 : (a.D > kThreads ? kThreads : ((a.D + 63) / 64) * 64));
  hipLaunchKernelGGL(decode_merge, dim3((unsigned)(a.B * a.Hq)), dim3(merge_threads),
                     (size_t)2 * stride * sizeof(float), s, p);
  return dkv_check_launch("dkv_decode_attention(merge)");
}
