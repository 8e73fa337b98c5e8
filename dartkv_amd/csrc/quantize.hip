// Quantize + pack kernels for the DartKV page layout (gfx950).
//
// * rows kernel: uniform group quantization along a row (value pages, and the
//   generic `quantize` API after its movedim), reference quantization.py:134-204.
// * key page kernel: one workgroup per (batch, kv-head, page); per-channel
//   token statistics, Dart channel selection (exact torch.topk order on one
//   lane), codes and LSB-first packing along tokens, reference mixed.py:119-244
//   and quantization.py:213-223 (axis=-2).
// * dequantize kernels: the reference's materialization chain
//   (quantization.py:96-109, mixed.py:72-94).
#include <hip/hip_runtime.h>

#include "dkv_capi_util.h"
#include "dkv_device.h"
#include "dkv_select.h"

using namespace dkv;

namespace {

constexpr int kThreads = 256;

// ---------------------------------------------------------------------------
// rows
// ---------------------------------------------------------------------------

struct RowsParams {
  const void* src;
  int64_t rows, n, row_stride, elem_stride;
  int64_t group, groups, packed_bytes;
  int bits, per_byte, src_dtype, meta_dtype;
  uint8_t* values;
  void* scale;
  void* zero;
};

__device__ __forceinline__ float row_elem(const RowsParams& p, int64_t r, int64_t i) {
  if (i >= p.n) i = p.n - 1;  // replicate the last element (quantization.py:174-177)
  return dev_load(p.src, r * p.row_stride + i * p.elem_stride, p.src_dtype);
}

__device__ __forceinline__ void group_stats(const RowsParams& p, int64_t r, int64_t g, float qmax, float* mn_out,
                                            float* scale_out) {
  float mn = row_elem(p, r, g * p.group), mx = mn;
  for (int64_t j = 1; j < p.group; ++j) {
    const float x = row_elem(p, r, g * p.group + j);
    mn = fminf(mn, x);
    mx = fmaxf(mx, x);
  }
  const float s = dev_group_scale(mn, mx, qmax, p.src_dtype);
  dev_store_meta(p.scale, r * p.groups + g, s, p.meta_dtype);
  dev_store_meta(p.zero, r * p.groups + g, mn, p.meta_dtype);
  *mn_out = mn;
  *scale_out = s;
}

// Groups that start on a byte boundary: one thread per (row, group).
__global__ void __launch_bounds__(kThreads) quantize_rows_aligned(RowsParams p) {
  const int64_t item = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (item >= p.rows * p.groups) return;
  const int64_t r = item / p.groups, g = item % p.groups;
  const float qmax = (float)((1 << p.bits) - 1);
  float mn, s;
  group_stats(p, r, g, qmax, &mn, &s);
  uint8_t* out = p.values + r * p.packed_bytes;
  const int64_t first = g * p.group;
  for (int64_t b = first / p.per_byte; b < (first + p.group) / p.per_byte; ++b) {
    uint32_t byte = 0;
    for (int j = 0; j < p.per_byte; ++j) {
      const int64_t i = b * p.per_byte + j;
      byte |= dev_group_code(row_elem(p, r, i), mn, s, qmax, p.src_dtype) << (j * p.bits);
    }
    out[b] = (uint8_t)byte;
  }
}

// Any group size: one thread per row walks the packed bytes in order.
__global__ void __launch_bounds__(kThreads) quantize_rows_serial(RowsParams p) {
  const int64_t r = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (r >= p.rows) return;
  const float qmax = (float)((1 << p.bits) - 1);
  const int64_t padded = p.groups * p.group;
  uint8_t* out = p.values + r * p.packed_bytes;
  float mn = 0.0f, s = 1.0f;
  int64_t cur = -1;
  for (int64_t b = 0; b < p.packed_bytes; ++b) {
    uint32_t byte = 0;
    for (int j = 0; j < p.per_byte; ++j) {
      const int64_t i = b * p.per_byte + j;
      if (i >= padded) break;
      const int64_t g = i / p.group;
      if (g != cur) {
        group_stats(p, r, g, qmax, &mn, &s);
        cur = g;
      }
      byte |= dev_group_code(row_elem(p, r, i), mn, s, qmax, p.src_dtype) << (j * p.bits);
    }
    out[b] = (uint8_t)byte;
  }
}

// ---------------------------------------------------------------------------
// key pages (quantized along tokens)
// ---------------------------------------------------------------------------

struct KeyParams {
  dkv_key_pages_args a;
  int64_t G;            // groups per channel
  int64_t nb;           // mixed: bytes per group
  int64_t pk;           // uniform: bytes per channel
};

__device__ __forceinline__ float key_elem(const KeyParams& k, int64_t b, int64_t h, int64_t page, int64_t t,
                                          int64_t c) {
  const dkv_key_pages_args& a = k.a;
  if (t >= a.page_tokens) t = a.page_tokens - 1;  // replicate the last token (mixed.py:196-197)
  const int64_t tok = page * a.page_tokens + t;
  return dev_load(a.src, b * a.sb + h * a.sh + tok * a.st + c * a.sd, (int)a.src_dtype);
}

// Token mean of f(x) over the page's real tokens with ATen's CPU cascade order
// (fp32 accumulate, 4 levels), then one division and one rounding to the
// source dtype.  mode 0: |x|; mode 1: rnd(rnd(x - mean)^2).
__device__ float channel_mean(const KeyParams& k, int64_t b, int64_t h, int64_t page, int64_t c, int mode,
                              float center) {
  const int64_t n = k.a.page_tokens;
  const int dt = (int)k.a.src_dtype;
  const int lp = cascade_level_power(n);
  const int64_t step = (int64_t)1 << lp, mask = step - 1;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  int64_t i = 0;
  auto term = [&](int64_t t) -> float {
    const float x = key_elem(k, b, h, page, t, c);
    if (mode == 0) return fabsf(x);
    const float d = dev_round_to(__fsub_rn(x, center), dt);
    return dev_round_to(__fmul_rn(d, d), dt);
  };
  for (; i + step <= n;) {
    for (int64_t j = 0; j < step; ++j, ++i) acc[0] = __fadd_rn(acc[0], term(i));
    for (int j = 1; j < 4; ++j) {
      acc[j] = __fadd_rn(acc[j], acc[j - 1]);
      acc[j - 1] = 0.f;
      if ((i & (mask << (j * lp))) != 0) break;
    }
  }
  for (; i < n; ++i) acc[0] = __fadd_rn(acc[0], term(i));
  for (int j = 1; j < 4; ++j) acc[0] = __fadd_rn(acc[0], acc[j]);
  return dev_round_to(__fdiv_rn(acc[0], (float)n), dt);
}

__global__ void __launch_bounds__(kThreads) quantize_key_pages_kernel(KeyParams k) {
  extern __shared__ unsigned char smem[];
  const dkv_key_pages_args& a = k.a;
  const int64_t bh = blockIdx.x, page = blockIdx.y;
  const int64_t b = bh / a.H, h = bh % a.H;
  const int64_t D = a.D;
  const int dt = (int)a.src_dtype, meta = (int)a.meta_dtype;
  const bool mixed = a.key_mode == DKV_KEY_MIXED;
  const int64_t K = mixed ? a.promoted : 0;

  float* score = (float*)smem;                       // [D]
  int32_t* slot = (int32_t*)(score + D);              // [D] promoted slot or -1
  int32_t* sel = slot + D;                            // [D] selected channel per slot
  SelItem* work = (SelItem*)(sel + D);                // [D]

  for (int64_t c = threadIdx.x; c < D; c += kThreads) slot[c] = -1;

  if (mixed && K > 0 && K < D && a.selection != DKV_SELECT_GIVEN) {
    for (int64_t c = threadIdx.x; c < D; c += kThreads) {
      if (a.selection == DKV_SELECT_MAGNITUDE) {
        score[c] = channel_mean(k, b, h, page, c, 0, 0.f);
      } else {
        // variance: mean(rnd(rnd(x - mean(x))^2)) (mixed.py:159-160)
        float m = 0.f;
        {
          const int64_t n = a.page_tokens;
          const int lp = cascade_level_power(n);
          const int64_t step = (int64_t)1 << lp, mask = step - 1;
          float acc[4] = {0.f, 0.f, 0.f, 0.f};
          int64_t i = 0;
          for (; i + step <= n;) {
            for (int64_t j = 0; j < step; ++j, ++i) acc[0] = __fadd_rn(acc[0], key_elem(k, b, h, page, i, c));
            for (int j = 1; j < 4; ++j) {
              acc[j] = __fadd_rn(acc[j], acc[j - 1]);
              acc[j - 1] = 0.f;
              if ((i & (mask << (j * lp))) != 0) break;
            }
          }
          for (; i < n; ++i) acc[0] = __fadd_rn(acc[0], key_elem(k, b, h, page, i, c));
          for (int j = 1; j < 4; ++j) acc[0] = __fadd_rn(acc[0], acc[j]);
          m = dev_round_to(__fdiv_rn(acc[0], (float)n), dt);
        }
        score[c] = channel_mean(k, b, h, page, c, 1, m);
      }
    }
    __syncthreads();
    if (threadIdx.x == 0) select_topk(score, (int)D, (int)K, work, sel);
    __syncthreads();
  } else if (mixed && K > 0) {
    for (int64_t j = threadIdx.x; j < K; j += kThreads)
      sel[j] = (K == D) ? (int32_t)j : a.given_idx[h * K + j];
    __syncthreads();
  }
  if (mixed && K > 0) {
    for (int64_t j = threadIdx.x; j < K; j += kThreads) {
      const int32_t ch = sel[j];
      if (ch >= 0 && ch < D) slot[ch] = (int32_t)j;
    }
    int32_t* idx_out = (int32_t*)((char*)a.idx + page * a.idx_page_stride) + bh * K;
    for (int64_t j = threadIdx.x; j < K; j += kThreads) idx_out[j] = sel[j];
    __syncthreads();
  }

  const int64_t G = k.G, group = a.group;
  uint8_t* low = a.low + page * a.low_page_stride;
  uint8_t* high = mixed ? a.high + page * a.high_page_stride : nullptr;
  void* scale = (char*)a.scale + page * a.scale_page_stride;
  void* zero = (char*)a.zero + page * a.zero_page_stride;
  const int bits = mixed ? 2 : (int)a.bits;
  const int per_byte = 8 / bits;

  for (int64_t c = threadIdx.x; c < D; c += kThreads) {
    const int32_t s_idx = slot[c];
    const float qmax = mixed ? (s_idx >= 0 ? 15.0f : 3.0f) : (float)((1 << a.bits) - 1);
    const int64_t meta_base = (bh * D + c) * G;
    float mn = 0.f, s = 1.f;
    if (mixed) {
      uint8_t* lrow = low + (bh * D + c) * G * k.nb;
      uint8_t* hrow = s_idx >= 0 ? high + (bh * K + s_idx) * G * k.nb : nullptr;
      for (int64_t g = 0; g < G; ++g) {
        mn = key_elem(k, b, h, page, g * group, c);
        float mx = mn;
        for (int64_t j = 1; j < group; ++j) {
          const float x = key_elem(k, b, h, page, g * group + j, c);
          mn = fminf(mn, x);
          mx = fmaxf(mx, x);
        }
        s = dev_group_scale(mn, mx, qmax, dt);
        dev_store_meta(scale, meta_base + g, s, meta);
        dev_store_meta(zero, meta_base + g, mn, meta);
        for (int64_t p = 0; p < k.nb; ++p) {
          uint32_t lo = 0, hi = 0;
          for (int j = 0; j < 4; ++j) {
            const int64_t w = p * 4 + j;
            if (w >= group) break;
            const uint32_t code = dev_group_code(key_elem(k, b, h, page, g * group + w, c), mn, s, qmax, dt);
            lo |= (code & 3u) << (2 * j);
            hi |= (code >> 2) << (2 * j);
          }
          lrow[g * k.nb + p] = (uint8_t)lo;
          if (hrow) hrow[g * k.nb + p] = (uint8_t)hi;
        }
      }
    } else {
      uint8_t* row = low + (bh * D + c) * k.pk;
      const int64_t padded = G * group;
      int64_t cur = -1;
      for (int64_t p = 0; p < k.pk; ++p) {
        uint32_t byte = 0;
        for (int j = 0; j < per_byte; ++j) {
          const int64_t i = p * per_byte + j;
          if (i >= padded) break;
          const int64_t g = i / group;
          if (g != cur) {
            mn = key_elem(k, b, h, page, g * group, c);
            float mx = mn;
            for (int64_t q = 1; q < group; ++q) {
              const float x = key_elem(k, b, h, page, g * group + q, c);
              mn = fminf(mn, x);
              mx = fmaxf(mx, x);
            }
            s = dev_group_scale(mn, mx, qmax, dt);
            dev_store_meta(scale, meta_base + g, s, meta);
            dev_store_meta(zero, meta_base + g, mn, meta);
            cur = g;
          }
          byte |= dev_group_code(key_elem(k, b, h, page, i, c), mn, s, qmax, dt) << (j * bits);
        }
        row[p] = (uint8_t)byte;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// dequantize
// ---------------------------------------------------------------------------

__global__ void __launch_bounds__(kThreads) dequantize_rows_kernel(const uint8_t* values, const void* scale,
                                                                   const void* zero, int meta, int64_t rows,
                                                                   int64_t n, int bits, int64_t group,
                                                                   int64_t groups, int64_t packed_bytes,
                                                                   void* out, int out_dt, int64_t out_stride) {
  const int64_t item = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (item >= rows * n) return;
  const int64_t r = item / n, i = item % n;
  const int per_byte = 8 / bits;
  const uint32_t code = (values[r * packed_bytes + i / per_byte] >> ((i % per_byte) * bits)) & ((1u << bits) - 1u);
  const int64_t g = i / group;
  const float v = dev_dequant(code, dev_load_meta(scale, r * groups + g, meta), dev_load_meta(zero, r * groups + g, meta),
                              meta, out_dt);
  dev_store(out, r * out_stride + i, v, out_dt);
}

__global__ void __launch_bounds__(kThreads) dequantize_mixed_kernel(const uint8_t* low, const uint8_t* high,
                                                                    const int32_t* idx, const void* scale,
                                                                    const void* zero, int meta, int64_t B,
                                                                    int64_t H, int64_t D, int64_t T,
                                                                    int64_t group, int64_t K, void* out,
                                                                    int out_dt) {
  extern __shared__ int32_t inv[];  // [D] slot of each channel for this block's (b, h)
  const int64_t bh = blockIdx.y;
  for (int64_t c = threadIdx.x; c < D; c += kThreads) inv[c] = -1;
  __syncthreads();
  for (int64_t j = threadIdx.x; j < K; j += kThreads) {
    const int32_t ch = idx[bh * K + j];
    if (ch >= 0 && ch < D) inv[ch] = (int32_t)j;
  }
  __syncthreads();
  const int64_t item = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (item >= T * D) return;
  const int64_t t = item / D, c = item % D;
  const int64_t G = (T + group - 1) / group, nb = (group + 3) / 4;
  const int64_t g = t / group, w = t % group;
  uint32_t code = (low[((bh * D + c) * G + g) * nb + w / 4] >> ((w % 4) * 2)) & 3u;
  const int32_t s = inv[c];
  if (s >= 0) code |= ((high[((bh * K + s) * G + g) * nb + w / 4] >> ((w % 4) * 2)) & 3u) << 2;
  const int64_t mi = (bh * D + c) * G + g;
  const float v = dev_dequant(code, dev_load_meta(scale, mi, meta), dev_load_meta(zero, mi, meta), meta, out_dt);
  dev_store(out, (bh * T + t) * D + c, v, out_dt);
}

bool valid_float_dtype(int64_t dt) { return dt == kF32 || dt == kF16 || dt == kBF16; }
bool valid_meta_dtype(int64_t dt) { return dt == kF32 || dt == kF16 || dt == kBF16 || dt == kF64; }
bool valid_bits(int64_t b) { return b == 2 || b == 4 || b == 8; }

}  // namespace

extern "C" int dkv_quantize_rows(const void* src, int src_dtype, int64_t rows, int64_t n, int64_t row_stride,
                                 int64_t elem_stride, int bits, int64_t group, uint8_t* values, void* scale,
                                 void* zero, int meta_dtype, void* stream) {
  DKV_CHECK(valid_float_dtype(src_dtype), DKV_ERR_DTYPE, "quantize expects a floating-point tensor (f32/f16/bf16)");
  DKV_CHECK(valid_meta_dtype(meta_dtype), DKV_ERR_DTYPE, "metadata dtype must be floating point");
  DKV_CHECK(valid_bits(bits), DKV_ERR_INVALID, "bits must be one of (2, 4, 8), got %d", bits);
  DKV_CHECK(group > 0, DKV_ERR_INVALID, "group_size must be a positive integer, got %lld", (long long)group);
  DKV_CHECK(n > 0 && rows >= 0, DKV_ERR_INVALID, "quantize does not support an empty final dimension");
  if (rows == 0) return DKV_OK;
  RowsParams p;
  p.src = src;
  p.rows = rows;
  p.n = n;
  p.row_stride = row_stride;
  p.elem_stride = elem_stride;
  p.group = group;
  p.groups = (n + group - 1) / group;
  p.bits = bits;
  p.per_byte = 8 / bits;
  const int64_t padded = p.groups * group;
  p.packed_bytes = (padded + p.per_byte - 1) / p.per_byte;
  p.src_dtype = src_dtype;
  p.meta_dtype = meta_dtype;
  p.values = values;
  p.scale = scale;
  p.zero = zero;
  hipStream_t s = (hipStream_t)stream;
  if (group % p.per_byte == 0) {
    const int64_t items = rows * p.groups;
    hipLaunchKernelGGL(quantize_rows_aligned, dim3((unsigned)((items + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                       s, p);
  } else {
    hipLaunchKernelGGL(quantize_rows_serial, dim3((unsigned)((rows + kThreads - 1) / kThreads)), dim3(kThreads), 0, s,
                       p);
  }
  return dkv_check_launch("dkv_quantize_rows");
}

extern "C" int dkv_quantize_key_pages(const dkv_key_pages_args* args, void* stream) {
  DKV_CHECK(args != nullptr, DKV_ERR_INVALID, "args is NULL");
  const dkv_key_pages_args& a = *args;
  DKV_CHECK(valid_float_dtype(a.src_dtype), DKV_ERR_DTYPE, "key_states must be floating point (f32/f16/bf16)");
  DKV_CHECK(valid_meta_dtype(a.meta_dtype), DKV_ERR_DTYPE, "metadata_dtype must be floating point");
  DKV_CHECK(a.B > 0 && a.H > 0 && a.D > 0 && a.page_tokens > 0 && a.n_pages >= 0, DKV_ERR_INVALID,
            "key_states sequence and head dimensions must be non-empty");
  DKV_CHECK(a.group > 0, DKV_ERR_INVALID, "group_size must be a positive integer");
  DKV_CHECK(a.key_mode == DKV_KEY_MIXED || a.key_mode == DKV_KEY_UNIFORM, DKV_ERR_INVALID, "unknown key_mode %lld",
            (long long)a.key_mode);
  if (a.key_mode == DKV_KEY_UNIFORM) {
    DKV_CHECK(valid_bits(a.bits), DKV_ERR_INVALID, "bits must be one of (2, 4, 8), got %lld", (long long)a.bits);
  } else {
    DKV_CHECK(a.promoted >= 0 && a.promoted <= a.D, DKV_ERR_INVALID, "promoted channels must be in [0, head_dim]");
    DKV_CHECK(a.selection >= 0 && a.selection <= 2, DKV_ERR_INVALID, "unknown channel selection");
    DKV_CHECK(a.selection != DKV_SELECT_GIVEN || a.promoted == 0 || a.promoted == a.D || a.given_idx != nullptr,
              DKV_ERR_INVALID, "given channel indices are required");
  }
  DKV_CHECK(a.B * a.H <= 0x7fffffffLL && a.n_pages <= 65535, DKV_ERR_UNSUPPORTED, "too many pages for one launch");
  if (a.n_pages == 0) return DKV_OK;
  KeyParams k;
  k.a = a;
  k.G = (a.page_tokens + a.group - 1) / a.group;
  k.nb = (a.group + 3) / 4;
  const int per_byte = a.key_mode == DKV_KEY_UNIFORM ? (int)(8 / a.bits) : 4;
  k.pk = (k.G * a.group + per_byte - 1) / per_byte;
  const size_t shmem = (size_t)a.D * (sizeof(float) + 2 * sizeof(int32_t) + sizeof(SelItem));
  DKV_CHECK(shmem <= 64 * 1024, DKV_ERR_UNSUPPORTED, "head_dim %lld is too large", (long long)a.D);
  hipLaunchKernelGGL(quantize_key_pages_kernel, dim3((unsigned)(a.B * a.H), (unsigned)a.n_pages), dim3(kThreads),
                     shmem, (hipStream_t)stream, k);
  return dkv_check_launch("dkv_quantize_key_pages");
}

extern "C" int dkv_dequantize_rows(const uint8_t* values, const void* scale, const void* zero, int meta_dtype,
                                   int64_t rows, int64_t n, int bits, int64_t group, void* out, int out_dtype,
                                   int64_t out_row_stride, void* stream) {
  DKV_CHECK(valid_meta_dtype(meta_dtype), DKV_ERR_DTYPE, "metadata dtype must be floating point");
  DKV_CHECK(valid_float_dtype(out_dtype), DKV_ERR_DTYPE, "output dtype must be f32/f16/bf16");
  DKV_CHECK(valid_bits(bits), DKV_ERR_INVALID, "bits must be one of (2, 4, 8)");
  DKV_CHECK(group > 0 && n > 0 && rows >= 0, DKV_ERR_INVALID, "bad dequantize shape");
  if (rows == 0) return DKV_OK;
  const int64_t groups = (n + group - 1) / group;
  const int per_byte = 8 / bits;
  const int64_t packed_bytes = (groups * group + per_byte - 1) / per_byte;
  const int64_t items = rows * n;
  hipLaunchKernelGGL(dequantize_rows_kernel, dim3((unsigned)((items + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                     (hipStream_t)stream, values, scale, zero, meta_dtype, rows, n, bits, group, groups, packed_bytes,
                     out, out_dtype, out_row_stride);
  return dkv_check_launch("dkv_dequantize_rows");
}

extern "C" int dkv_dequantize_mixed(const uint8_t* low, const uint8_t* high, const int32_t* idx, const void* scale,
                                    const void* zero, int meta_dtype, int64_t B, int64_t H, int64_t D, int64_t tokens,
                                    int64_t group, int64_t promoted, void* out, int out_dtype, void* stream) {
  DKV_CHECK(valid_meta_dtype(meta_dtype), DKV_ERR_DTYPE, "metadata dtype must be floating point");
  DKV_CHECK(valid_float_dtype(out_dtype), DKV_ERR_DTYPE, "output dtype must be f32/f16/bf16");
  DKV_CHECK(B > 0 && H > 0 && D > 0 && tokens > 0 && group > 0, DKV_ERR_INVALID, "bad dequantize shape");
  DKV_CHECK(promoted >= 0 && promoted <= D, DKV_ERR_INVALID, "bad promoted channel count");
  DKV_CHECK(D <= 16384 && B * H <= 65535, DKV_ERR_UNSUPPORTED, "shape too large for dkv_dequantize_mixed");
  const int64_t items = tokens * D;
  hipLaunchKernelGGL(dequantize_mixed_kernel, dim3((unsigned)((items + kThreads - 1) / kThreads), (unsigned)(B * H)),
                     dim3(kThreads), (size_t)D * sizeof(int32_t), (hipStream_t)stream, low, high, idx, scale, zero,
                     meta_dtype, B, H, D, tokens, group, promoted, out, out_dtype);
  return dkv_check_launch("dkv_dequantize_mixed");
}
