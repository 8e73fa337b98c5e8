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

#include <algorithm>

#include "dkv_capi_util.h"
#include "dkv_copy.h"
#include "dkv_device.h"
#include "dkv_select.h"
#include "dkv_select_wave.h"

using namespace dkv;

namespace {

constexpr int kThreads = 256;

// Group minimum / maximum that propagate NaN (v_minimum3_f32 / v_maximum3_f32
// on gfx950; on finite values they equal fminf / fmaxf).  A group holding a
// NaN or an infinity therefore ends with a non-finite min or max, and
// flag_nonfinite reports it: the reference rejects such inputs
// (quantization.py:159-160, mixed.py:187-188).
__device__ __forceinline__ float nmin(float a, float b) { return __builtin_elementwise_minimum(a, b); }
__device__ __forceinline__ float nmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ double nmin(double a, double b) { return __builtin_elementwise_minimum(a, b); }
__device__ __forceinline__ double nmax(double a, double b) { return __builtin_elementwise_maximum(a, b); }

// flag (may be NULL) := 1 when a group's min or max is not finite.  Every
// writer stores the same value, with a vector store.
template <typename A>
__device__ __forceinline__ void flag_nonfinite(uint32_t* flag, A mn, A mx) {
  if (flag != nullptr && !(__builtin_isfinite(mn) && __builtin_isfinite(mx))) *flag = 1u;
}

// The generic (any layout) kernels below run in A = float for fp32, fp16 and
// bf16 sources (each op rounded to the source dtype) and in A = double for
// float64 sources: the reference quantizes in the source dtype
// (quantization.py:179-186), so a float64 tensor is quantized in float64.
template <typename A>
__device__ __forceinline__ A src_elem(const void* base, int64_t index, int dt);
template <>
__device__ __forceinline__ float src_elem<float>(const void* base, int64_t index, int dt) {
  return dev_load(base, index, dt);
}
template <>
__device__ __forceinline__ double src_elem<double>(const void* base, int64_t index, int) {
  return ((const double*)base)[index];
}

// ---------------------------------------------------------------------------
// rows
// ---------------------------------------------------------------------------

struct RowsParams {
  const void* src;
  int64_t rows, n, row_stride, elem_stride;
  // rows come in blocks of block_rows: row r = blk * block_rows + i starts at
  // blk * block_stride + i * row_stride (one block: block_rows = rows)
  int64_t blocks, block_rows, block_stride;
  int64_t group, groups, packed_bytes;
  int bits, per_byte, src_dtype, meta_dtype;
  uint8_t* values;
  void* scale;
  void* zero;
  uint32_t* nonfinite;  // optional flag, set when a group holds a non-finite value
  // output placement: source row blk * block_rows + i is written to output row
  // blk * out_block_rows + out_row0 + i
  int64_t out_block_rows, out_row0;
};

__device__ __forceinline__ int64_t out_row(const RowsParams& p, int64_t r) {
  return (r / p.block_rows) * p.out_block_rows + p.out_row0 + r % p.block_rows;
}

template <typename A>
__device__ __forceinline__ A row_elem(const RowsParams& p, int64_t r, int64_t i) {
  if (i >= p.n) i = p.n - 1;  // replicate the last element (quantization.py:174-177)
  const int64_t row = (r / p.block_rows) * p.block_stride + (r % p.block_rows) * p.row_stride;
  return src_elem<A>(p.src, row + i * p.elem_stride, p.src_dtype);
}

template <typename A>
__device__ __forceinline__ void group_stats(const RowsParams& p, int64_t r, int64_t g, A qmax, A* mn_out,
                                            A* scale_out) {
  A mn = row_elem<A>(p, r, g * p.group), mx = mn;
  for (int64_t j = 1; j < p.group; ++j) {
    const A x = row_elem<A>(p, r, g * p.group + j);
    mn = nmin(mn, x);
    mx = nmax(mx, x);
  }
  flag_nonfinite(p.nonfinite, mn, mx);
  const A s = dev_group_scale(mn, mx, qmax, p.src_dtype);
  const int64_t o = out_row(p, r);
  dev_store_meta(p.scale, o * p.groups + g, s, p.meta_dtype);
  dev_store_meta(p.zero, o * p.groups + g, mn, p.meta_dtype);
  *mn_out = mn;
  *scale_out = s;
}

// Groups that start on a byte boundary: one thread per (row, group).
template <typename A>
__global__ void __launch_bounds__(kThreads) quantize_rows_aligned(RowsParams p) {
  const int64_t item = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (item >= p.rows * p.groups) return;
  const int64_t r = item / p.groups, g = item % p.groups;
  const A qmax = (A)((1 << p.bits) - 1);
  A mn, s;
  group_stats<A>(p, r, g, qmax, &mn, &s);
  uint8_t* out = p.values + out_row(p, r) * p.packed_bytes;
  const int64_t first = g * p.group;
  for (int64_t b = first / p.per_byte; b < (first + p.group) / p.per_byte; ++b) {
    uint32_t byte = 0;
    for (int j = 0; j < p.per_byte; ++j) {
      const int64_t i = b * p.per_byte + j;
      byte |= dev_group_code(row_elem<A>(p, r, i), mn, s, qmax, p.src_dtype) << (j * p.bits);
    }
    out[b] = (uint8_t)byte;
  }
}

// Rounding to the source dtype with the hardware conversions (round to
// nearest even): one v_cvt_pk_bf16_f32 / v_cvt_f16_f32 and its widening.
template <int SRC>
__device__ __forceinline__ float src_round(float x) {
  if (SRC == kBF16) return (float)(__bf16)x;
  if (SRC == kF16) return (float)(_Float16)x;
  return x;
}

// Four quotients q of the exact chain (each x - min rounded, divided by the
// group scale, rounded) to their codes clamp(rint(q), 0, qmax), one byte each
// (byte j of the result), with v_cvt_pk_u8_f32: it rounds half to even and
// clamps to [0, 255] (checked against rint on the device over every bf16 value
// in [-4, 300] and the fp32 neighbours of half-integers).  The chain never
// gives q < 0 (x >= min), and q < qmax + 1/2: the scale s is range / qmax
// rounded (relative error at most 2^-9 for bf16, less for fp16 and fp32), so
// q <= qmax (1 + 2^-8) + one rounding, below qmax + 1/2 for qmax 3 and 15; for
// qmax 255 the instruction's own clamp is the chain's.
__device__ __forceinline__ uint32_t codes_as_bytes(const float (&q)[4]) {
  uint32_t r = __builtin_amdgcn_cvt_pk_u8_f32(q[0], 0u, 0u);
  r = __builtin_amdgcn_cvt_pk_u8_f32(q[1], 1u, r);
  r = __builtin_amdgcn_cvt_pk_u8_f32(q[2], 2u, r);
  return __builtin_amdgcn_cvt_pk_u8_f32(q[3], 3u, r);
}
// Codes into byte planes, so packing needs no per-byte shuffling: the
// v_cvt_pk_u8_f32 that forms a code (the same one instruction per code as
// codes_as_bytes) writes it at the byte where the packed layout wants it.
//
// 2-bit fields, 16 codes per dword (code i at bits 2i, LSB first): plane t
// holds code 4h + t at byte h, for quotients q of codes 4h .. 4h + 3.
__device__ __forceinline__ void codes_to_planes2(const float (&q)[4], int h, uint32_t (&plane)[4]) {
#pragma unroll
  for (int t = 0; t < 4; ++t) plane[t] = __builtin_amdgcn_cvt_pk_u8_f32(q[t], (uint32_t)h, plane[t]);
}
// The 16 fields from codes below 4: byte h = code 4h | code 4h+1 << 2 | ...
__device__ __forceinline__ uint32_t pack2(const uint32_t (&plane)[4]) {
  return plane[0] | (plane[1] << 2) | (plane[2] << 4) | (plane[3] << 6);
}
// Codes below 16 (Dart keys: 4-bit codes of promoted channels, 2-bit ones
// elsewhere): the fields of their low two bits and of their high two bits.
// (m & a) | (~m & b) is one v_bfi_b32; bits a shift carries into a
// neighbouring field are overwritten by the outer selections.
__device__ __forceinline__ uint32_t bit_select(uint32_t m, uint32_t a, uint32_t b) { return (m & a) | (~m & b); }
__device__ __forceinline__ uint32_t pack2_low(const uint32_t (&plane)[4]) {
  return bit_select(0x03030303u, plane[0],
                    bit_select(0x0c0c0c0cu, plane[1] << 2, bit_select(0x30303030u, plane[2] << 4, plane[3] << 6)));
}
__device__ __forceinline__ uint32_t pack2_high(const uint32_t (&plane)[4]) {
  return bit_select(0x03030303u, plane[0] >> 2,
                    bit_select(0x0c0c0c0cu, plane[1], bit_select(0x30303030u, plane[2] << 2, plane[3] << 4)));
}
// 4-bit fields, 8 codes per dword (code i at bits 4i): plane t % 2 holds code
// 4h + t at byte 2h + t / 2 (h = 0, 1), so the dword is even | odd << 4.
__device__ __forceinline__ void codes_to_planes4(const float (&q)[4], int h, uint32_t (&plane)[2]) {
#pragma unroll
  for (int t = 0; t < 4; ++t)
    plane[t & 1] = __builtin_amdgcn_cvt_pk_u8_f32(q[t], (uint32_t)(2 * h + (t >> 1)), plane[t & 1]);
}
__device__ __forceinline__ uint32_t pack4(const uint32_t (&plane)[2]) { return plane[0] | (plane[1] << 4); }

// fp32 a / b rounded to nearest, given y = RN(1 / b): q = RN(a y) is within
// one ulp of a / b, the residual a - b q is exact with an fma, and
// RN(q + (a - b q) y) is the correctly rounded quotient (Markstein's
// theorem; no overflow or underflow for quotients of group-relative values).
__device__ __forceinline__ float div_rn(float a, float b, float y) {
  const float q = a * y;
  const float r = __builtin_fmaf(-q, b, a);
  return __builtin_fmaf(r, y, q);
}

// Two values rounded to the source dtype at once: for bf16 one packed
// conversion (v_cvt_pk_bf16_f32, nearest-even like the single one) and two
// unpacks instead of two conversions and two unpacks.
template <int SRC>
__device__ __forceinline__ void src_round2(float& a, float& b) {
  if (SRC == kBF16) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    const uint32_t u = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
    a = __builtin_bit_cast(float, u << 16);
    b = __builtin_bit_cast(float, u & 0xffff0000u);
  } else {
    a = src_round<SRC>(a);
    b = src_round<SRC>(b);
  }
}

// The exact chain's quotients of four elements: round(round(x - mn) / s),
// y = RN(1 / s).  For fp32 sources the division is div_rn.  For bf16 and fp16
// sources (d and s 16-bit values) it is one product: rint(round_src(RN(d y)))
// equals rint(round_src(RN(d / s))) for every 16-bit d >= 0 and s >= 3.8e-7
// (the smallest scale the eps clamp allows) with d / s < 256, checked
// exhaustively on the host (tests/quotient/chain_quotient.c); the rounded
// quotients differ in rare cases, never in the integer they round to, and
// only that integer (the code) is kept.
template <int SRC>
__device__ __forceinline__ void chain_quotients4(const float* x, float mn, float s, float y, float (&q)[4]) {
  float d[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) d[j] = x[j] - mn;
  src_round2<SRC>(d[0], d[1]);
  src_round2<SRC>(d[2], d[3]);
#pragma unroll
  for (int j = 0; j < 4; ++j) q[j] = SRC == kF32 ? div_rn(d[j], s, y) : d[j] * y;
  src_round2<SRC>(q[0], q[1]);
  src_round2<SRC>(q[2], q[3]);
}


// The group scale of dev_group_scale (round(round(max - min) / qmax) in the
// source dtype, range clamped below by eps) with the division by qmax as
// div_rn against y = RN(1 / qmax).  For qmax 3, 15 and 255 that equals the
// IEEE quotient for every positive finite fp32 range (checked exhaustively
// on the host); an infinite range keeps the IEEE result, infinity.
template <int SRC>
__device__ __forceinline__ float rows_group_scale(float mn, float mx, float qmax, float inv_qmax) {
  float range = src_round<SRC>(mx - mn);
  if (!(range >= quant_eps(SRC))) range = quant_eps(SRC);
  const float d = range == INFINITY ? INFINITY : div_rn(range, qmax, inv_qmax);
  return src_round<SRC>(d);
}

// Contiguous rows, groups of E * L elements (E = 8 or 16 elements per lane, L =
// 1..64 lanes, a power of two) that tile the row exactly: every lane owns E
// consecutive elements (16-byte loads for 16-bit sources), the L lanes of a
// group reduce min/max with cross-lane shuffles, and every lane stores its E
// codes packed.  A wave's loads and stores are contiguous.  The source dtype
// is a template argument, so the per-element chain (subtract, round, divide,
// round, rint, clamp) has no branches; the division is one reciprocal per
// group and three operations per element.  The per-group work (shuffles,
// scale, reciprocal, metadata stores) is one instruction stream per lane
// whatever E is, so 16 elements per lane spend about a quarter fewer VALU
// instructions per element than 8.  Workgroup (bx, by) of a gx x gy grid: y
// strides over row blocks, x over the lanes of one block, kRowChunks chunks of
// kThreads lanes per step: a lane issues the loads of all its chunks before it
// computes (one chunk per lane left each wave with one 16-byte load in flight
// per lane, and the kernel waiting on memory latency).
constexpr int kRowChunks = 2;

// Elements i0 .. i0 + 7 of a source row as fp32.
template <int SRC>
__device__ __forceinline__ void load_row8(const RowsParams& p, int64_t src_row, int64_t i0, float* x) {
  if (SRC == kF32) {
    const float4* src = (const float4*)((const float*)p.src + src_row + i0);
    const float4 a = src[0], b = src[1];
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
  } else {
    const uint4 w = *(const uint4*)((const uint16_t*)p.src + src_row + i0);
    const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint16_t bits = (uint16_t)(ww[j / 2] >> (16 * (j % 2)));
      x[j] = SRC == kBF16 ? bf16_to_f32(bits) : (float)__builtin_bit_cast(_Float16, bits);
    }
  }
}

template <int BITS, int SRC, int E>
__device__ __forceinline__ void rows_vec_body(const RowsParams& p, int lanes_per_group, int row_shift, int64_t bx,
                                              int64_t by, int64_t gx, int64_t gy) {
  static_assert(E == 8 || E == 16, "8 or 16 elements per lane");
  // row_shift = log2(lanes per row) when that is a power of two (no 64-bit division)
  const int64_t lanes_per_row = p.n / E;
  const int64_t total = p.block_rows * lanes_per_row;
  const float qmax = (float)((1 << BITS) - 1);
  constexpr float inv_qmax = 1.0f / (float)((1 << BITS) - 1);  // RN(1 / qmax), folded at compile time
  const int group_shift = __builtin_ctz((unsigned)lanes_per_group);
  const int lane = threadIdx.x & 63;
  constexpr int64_t kStep = (int64_t)kThreads * kRowChunks;
  for (int64_t blk = by; blk < p.blocks; blk += gy)
  for (int64_t v0 = bx * kStep + threadIdx.x; v0 - lane < total; v0 += gx * kStep) {
    // whole waves stay in the loop so the shuffles see every lane of a group
    int64_t r[kRowChunks];   // row within the block
    int li[kRowChunks];      // lane item within the row: elements E li .. E li + E - 1
    float x[kRowChunks][E];
#pragma unroll
    for (int u = 0; u < kRowChunks; ++u) {
      const int64_t v = v0 + u * kThreads;
      r[u] = 0;
      li[u] = 0;
      if (v < total) {
        r[u] = row_shift >= 0 ? v >> row_shift : v / lanes_per_row;
        li[u] = (int)(v - r[u] * lanes_per_row);
        const int64_t row = blk * p.block_stride + r[u] * p.row_stride;
#pragma unroll
        for (int c = 0; c < E / 8; ++c) load_row8<SRC>(p, row, (int64_t)E * li[u] + 8 * c, &x[u][8 * c]);
      } else {
#pragma unroll
        for (int j = 0; j < E; ++j) x[u][j] = 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < kRowChunks; ++u) {
      const int64_t v = v0 + u * kThreads;
      if (v - lane >= total) break;  // the whole wave is past the block
      const bool active = v < total;
      float mn = x[u][0], mx = x[u][0];
#pragma unroll
      for (int j = 1; j < E; ++j) {
        mn = nmin(mn, x[u][j]);
        mx = nmax(mx, x[u][j]);
      }
      for (int off = 1; off < lanes_per_group; off <<= 1) {
        mn = nmin(mn, __shfl_xor(mn, off, 64));
        mx = nmax(mx, __shfl_xor(mx, off, 64));
      }
      if (!active) continue;
      const int64_t ro = r[u] + blk * p.out_block_rows + p.out_row0;  // output row
      const float s = rows_group_scale<SRC>(mn, mx, qmax, inv_qmax);
      const float y = __fdiv_rn(1.0f, s);
      if ((li[u] & (lanes_per_group - 1)) == 0) {  // the group's first lane (groups are power-of-two lanes)
        const int64_t g = li[u] >> group_shift;
        dev_store_meta(p.scale, ro * p.groups + g, s, p.meta_dtype);
        dev_store_meta(p.zero, ro * p.groups + g, mn, p.meta_dtype);
        flag_nonfinite(p.nonfinite, mn, mx);
      }
      // codes four at a time, each written by its conversion at its byte of
      // the packed layout (codes_to_planes2 / codes_to_planes4; 8-bit codes
      // are bytes in order), then the fields combined; codes are at most qmax
      uint8_t* out = p.values + ro * p.packed_bytes + (int64_t)li[u] * (E * BITS / 8);
      if (BITS == 2) {
        uint32_t plane[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int h = 0; h < E / 4; ++h) {
          float q[4];
          chain_quotients4<SRC>(&x[u][4 * h], mn, s, y, q);
          codes_to_planes2(q, h, plane);
        }
        const uint32_t w = pack2(plane);
        if (E == 8) *(uint16_t*)out = (uint16_t)w;
        else *(uint32_t*)out = w;
      } else if (BITS == 4) {
        uint32_t w[E / 8];
#pragma unroll
        for (int k = 0; k < E / 8; ++k) {
          uint32_t plane[2] = {0u, 0u};
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            float q[4];
            chain_quotients4<SRC>(&x[u][8 * k + 4 * h], mn, s, y, q);
            codes_to_planes4(q, h, plane);
          }
          w[k] = pack4(plane);
        }
        if (E == 8) *(uint32_t*)out = w[0];
        else *(uint2*)out = make_uint2(w[0], w[1]);
      } else {
        uint32_t bytes[E / 4];
#pragma unroll
        for (int h = 0; h < E / 4; ++h) {
          float q[4];
          chain_quotients4<SRC>(&x[u][4 * h], mn, s, y, q);
          bytes[h] = codes_as_bytes(q);
        }
        if (E == 8) *(uint2*)out = make_uint2(bytes[0], bytes[1]);
        else *(uint4*)out = make_uint4(bytes[0], bytes[1], bytes[2], bytes[3]);
      }
    }
  }
}

template <int BITS, int SRC, int E>
__global__ void __launch_bounds__(kThreads) quantize_rows_vec(RowsParams p, int lanes_per_group, int row_shift) {
  rows_vec_body<BITS, SRC, E>(p, lanes_per_group, row_shift, blockIdx.x, blockIdx.y, gridDim.x, gridDim.y);
}

// Any group size: one thread per row walks the packed bytes in order.
template <typename A>
__global__ void __launch_bounds__(kThreads) quantize_rows_serial(RowsParams p) {
  const int64_t r = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (r >= p.rows) return;
  const A qmax = (A)((1 << p.bits) - 1);
  const int64_t padded = p.groups * p.group;
  uint8_t* out = p.values + out_row(p, r) * p.packed_bytes;
  A mn = 0, s = 1;
  int64_t cur = -1;
  for (int64_t b = 0; b < p.packed_bytes; ++b) {
    uint32_t byte = 0;
    for (int j = 0; j < p.per_byte; ++j) {
      const int64_t i = b * p.per_byte + j;
      if (i >= padded) break;
      const int64_t g = i / p.group;
      if (g != cur) {
        group_stats<A>(p, r, g, qmax, &mn, &s);
        cur = g;
      }
      byte |= dev_group_code(row_elem<A>(p, r, i), mn, s, qmax, p.src_dtype) << (j * p.bits);
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

// One wave64 as the lane model of dkv_select_wave.h: lane l owns positions l
// and l + 64; LDS written by one lane is read by another only across sync().
struct DeviceWave {
  int lane;
  template <class T>
  struct PerPos {
    T v[2];
    __device__ T& at(int, int h) { return v[h]; }
  };
  template <class F>
  __device__ void each(F fn) {
    fn(lane, 0);
    fn(lane + 64, 1);
  }
  template <class F>
  __device__ uint64_t ballot(F pred, int h) {
    return __ballot(pred(lane + 64 * h));
  }
  __device__ bool first_lane() const { return lane == 0; }
  __device__ void sync() const {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
};

// Promoted channels of n <= 128 scores in torch.topk(sorted=True) order,
// ties included, by the calling wave (every lane of it calls): packed (rank,
// index) words, the wave-parallel selection, and lane 0 alone on the serial
// form where libstdc++ takes heap select or partial_sort.  wb.stack holds
// 3 * kSelectStack ints.  The K indices go to `out` (LDS or global memory).
constexpr int kSelectStack = 16;  // >= 2 floor(log2(128)) + 1
static_assert(kSelectStack >= kWaveSelStack, "one stack serves both forms");

__device__ __forceinline__ void wave_select_topk(const float* score, int n, int K, int lane, const WaveSelBuffers& wb,
                                                 int32_t* out) {
  DeviceWave w{lane};
  auto fill = [&]() {
    w.each([&](int x, int) {
      if (x < n) wb.a[x] = (sel_rank(score[x], score, n) << 7) | (uint32_t)x;
    });
    w.sync();
  };
  fill();
  if (!wsel_topk(wb, w, n, K)) {
    fill();
    if (lane == 0) sel_topk(n, K, PtrArray<PackedItem>{(PackedItem*)wb.a}, PtrArray<int>{wb.stack}, kSelectStack);
    w.sync();
  }
  w.each([&](int x, int) {
    if (x < K) out[x] = (int32_t)(wb.a[x] & 127u);
  });
}

template <typename A>
__device__ __forceinline__ A key_elem(const KeyParams& k, int64_t b, int64_t h, int64_t page, int64_t t, int64_t c) {
  const dkv_key_pages_args& a = k.a;
  if (t >= a.page_tokens) t = a.page_tokens - 1;  // replicate the last token (mixed.py:196-197)
  const int64_t tok = page * a.page_tokens + t;
  return src_elem<A>(a.src, b * a.sb + h * a.sh + tok * a.st + c * a.sd, (int)a.src_dtype);
}

// One op of the generic kernels' arithmetic, rounded to nearest in A (and, for
// A = float, then to the 16-bit source dtype by a_round).
__device__ __forceinline__ float a_add(float x, float y) { return __fadd_rn(x, y); }
__device__ __forceinline__ double a_add(double x, double y) { return __dadd_rn(x, y); }
__device__ __forceinline__ float a_sub(float x, float y) { return __fsub_rn(x, y); }
__device__ __forceinline__ double a_sub(double x, double y) { return __dsub_rn(x, y); }
__device__ __forceinline__ float a_mul(float x, float y) { return __fmul_rn(x, y); }
__device__ __forceinline__ double a_mul(double x, double y) { return __dmul_rn(x, y); }
__device__ __forceinline__ float a_div(float x, float y) { return __fdiv_rn(x, y); }
__device__ __forceinline__ double a_div(double x, double y) { return __ddiv_rn(x, y); }
__device__ __forceinline__ float a_abs(float x) { return fabsf(x); }
__device__ __forceinline__ double a_abs(double x) { return fabs(x); }
__device__ __forceinline__ float a_round(float x, int dt) { return dev_round_to(x, dt); }
__device__ __forceinline__ double a_round(double x, int) { return x; }

// Token mean of f(x) over the page's real tokens with ATen's CPU cascade order
// (4 levels, accumulated in fp32 for fp32/fp16/bf16 sources and in double for
// float64 ones: ATen's accumulate type of each), then one division and one
// rounding to the source dtype.  mode 0: |x|; mode 1: rnd(rnd(x - center)^2);
// mode 2: x.
template <typename A>
__device__ A channel_mean(const KeyParams& k, int64_t b, int64_t h, int64_t page, int64_t c, int mode, A center) {
  const int64_t n = k.a.page_tokens;
  const int dt = (int)k.a.src_dtype;
  const int lp = cascade_level_power(n);
  const int64_t step = (int64_t)1 << lp, mask = step - 1;
  A acc[4] = {0, 0, 0, 0};
  int64_t i = 0;
  auto term = [&](int64_t t) -> A {
    const A x = key_elem<A>(k, b, h, page, t, c);
    if (mode == 0) return a_abs(x);
    if (mode == 2) return x;
    const A d = a_round(a_sub(x, center), dt);
    return a_round(a_mul(d, d), dt);
  };
  for (; i + step <= n;) {
    for (int64_t j = 0; j < step; ++j, ++i) acc[0] = a_add(acc[0], term(i));
    for (int j = 1; j < 4; ++j) {
      acc[j] = a_add(acc[j], acc[j - 1]);
      acc[j - 1] = 0;
      if ((i & (mask << (j * lp))) != 0) break;
    }
  }
  for (; i < n; ++i) acc[0] = a_add(acc[0], term(i));
  for (int j = 1; j < 4; ++j) acc[0] = a_add(acc[0], acc[j]);
  return a_round(a_div(acc[0], (A)n), dt);
}

// Shared memory of quantize_key_pages_kernel<A> for head_dim D.
template <typename A>
size_t key_generic_smem(int64_t D) {
  return (size_t)D * (sizeof(float) + 2 * sizeof(int32_t) + sizeof(SelItem) + (sizeof(A) == 8 ? sizeof(double) : 0));
}

template <typename A>
__global__ void __launch_bounds__(kThreads) quantize_key_pages_kernel(KeyParams k) {
  extern __shared__ unsigned char smem[];
  const dkv_key_pages_args& a = k.a;
  const int64_t bh = blockIdx.x, page = blockIdx.y;
  const int64_t b = bh / a.H, h = bh % a.H;
  const int64_t D = a.D;
  const int dt = (int)a.src_dtype, meta = (int)a.meta_dtype;
  const bool mixed = a.key_mode == DKV_KEY_MIXED;
  const int64_t K = mixed ? a.promoted : 0;
  constexpr bool kDouble = sizeof(A) == 8;

  // [D] double scores (float64 sources only), then [D] float selection keys
  double* dscore = (double*)smem;
  float* score = (float*)(smem + (kDouble ? D * sizeof(double) : 0));
  int32_t* slot = (int32_t*)(score + D);              // [D] promoted slot or -1
  int32_t* sel = slot + D;                            // [D] selected channel per slot
  SelItem* work = (SelItem*)(sel + D);                // [D]

  for (int64_t c = threadIdx.x; c < D; c += kThreads) slot[c] = -1;

  if (mixed && K > 0 && K < D && a.selection != DKV_SELECT_GIVEN) {
    for (int64_t c = threadIdx.x; c < D; c += kThreads) {
      A sc;
      if (a.selection == DKV_SELECT_MAGNITUDE) {
        sc = channel_mean<A>(k, b, h, page, c, 0, A(0));
      } else {
        // variance: mean(rnd(rnd(x - mean(x))^2)) (mixed.py:159-160)
        sc = channel_mean<A>(k, b, h, page, c, 1, channel_mean<A>(k, b, h, page, c, 2, A(0)));
      }
      if (kDouble) {
        dscore[c] = (double)sc;
      } else {
        score[c] = (float)sc;
      }
    }
    __syncthreads();
    if (kDouble) {
      // The selection compares scores only, so each double score is replaced
      // by its rank among the page's scores (D for NaN, which ranks first):
      // equal scores get equal ranks and the order is kept, so the selection
      // on the ranks (exact in float) makes the same steps as on the doubles.
      for (int64_t c = threadIdx.x; c < D; c += kThreads) {
        const double v = dscore[c];
        int64_t r = 0;
        if (v != v) {
          r = D;
        } else {
          for (int64_t j = 0; j < D; ++j) r += dscore[j] < v ? 1 : 0;
        }
        score[c] = (float)r;
      }
      __syncthreads();
    }
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
    const A qmax = mixed ? (s_idx >= 0 ? A(15) : A(3)) : (A)((1 << a.bits) - 1);
    const int64_t meta_base = (bh * D + c) * G;
    A mn = 0, s = 1;
    if (mixed) {
      uint8_t* lrow = low + (bh * D + c) * G * k.nb;
      uint8_t* hrow = s_idx >= 0 ? high + (bh * K + s_idx) * G * k.nb : nullptr;
      for (int64_t g = 0; g < G; ++g) {
        mn = key_elem<A>(k, b, h, page, g * group, c);
        A mx = mn;
        for (int64_t j = 1; j < group; ++j) {
          const A x = key_elem<A>(k, b, h, page, g * group + j, c);
          mn = nmin(mn, x);
          mx = nmax(mx, x);
        }
        flag_nonfinite(a.nonfinite, mn, mx);
        s = dev_group_scale(mn, mx, qmax, dt);
        dev_store_meta(scale, meta_base + g, s, meta);
        dev_store_meta(zero, meta_base + g, mn, meta);
        for (int64_t p = 0; p < k.nb; ++p) {
          uint32_t lo = 0, hi = 0;
          for (int j = 0; j < 4; ++j) {
            const int64_t w = p * 4 + j;
            if (w >= group) break;
            const uint32_t code = dev_group_code(key_elem<A>(k, b, h, page, g * group + w, c), mn, s, qmax, dt);
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
            mn = key_elem<A>(k, b, h, page, g * group, c);
            A mx = mn;
            for (int64_t q = 1; q < group; ++q) {
              const A x = key_elem<A>(k, b, h, page, g * group + q, c);
              mn = nmin(mn, x);
              mx = nmax(mx, x);
            }
            flag_nonfinite(a.nonfinite, mn, mx);
            s = dev_group_scale(mn, mx, qmax, dt);
            dev_store_meta(scale, meta_base + g, s, meta);
            dev_store_meta(zero, meta_base + g, mn, meta);
            cur = g;
          }
          byte |= dev_group_code(key_elem<A>(k, b, h, page, i, c), mn, s, qmax, dt) << (j * bits);
        }
        row[p] = (uint8_t)byte;
      }
    }
  }
}

// LDS-tiled key page kernel for 16-bit sources with unit channel stride:
// one workgroup per (batch * head, page).  The page's [T][D] tile is staged
// in LDS with 16-byte loads (rows padded by 4 bytes so a column read is
// conflict-free), per-channel statistics and the channel scores are read from
// LDS (same reduction order as channel_mean), the top-k selection runs on one
// lane, codes are packed into LDS buffers, and the packed page is written out
// with 16-byte stores.
constexpr int kKeyTileMaxBytes = 48 * 1024;

__host__ __device__ inline int key_tile_row_bytes(int D) { return 2 * D + 4; }

__device__ __forceinline__ float tile_elem(const uint8_t* tile, int rs, int T, int t, int c, int dt) {
  if (t >= T) t = T - 1;  // replicate the last token (mixed.py:196-197, quantization.py:174-177)
  const uint16_t bits = *(const uint16_t*)(tile + t * rs + 2 * c);
  return dt == kBF16 ? bf16_to_f32(bits) : (float)__builtin_bit_cast(_Float16, bits);
}

// Token mean of f(x) over the T real tokens of channel c (mode 0: |x|;
// mode 1: rnd(rnd(x - center)^2)) with ATen's CPU cascade order.
__device__ float tile_channel_mean(const uint8_t* tile, int rs, int T, int c, int dt, int mode, float center) {
  const int lp = cascade_level_power(T);
  const int step = 1 << lp, mask = step - 1;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  int i = 0;
  auto term = [&](int t) -> float {
    const float x = tile_elem(tile, rs, T, t, c, dt);
    if (mode == 0) return fabsf(x);
    if (mode == 2) return x;
    const float d = dev_round_to(__fsub_rn(x, center), dt);
    return dev_round_to(__fmul_rn(d, d), dt);
  };
  for (; i + step <= T;) {
    for (int j = 0; j < step; ++j, ++i) acc[0] = __fadd_rn(acc[0], term(i));
    for (int j = 1; j < 4; ++j) {
      acc[j] = __fadd_rn(acc[j], acc[j - 1]);
      acc[j - 1] = 0.f;
      if ((i & (mask << (j * lp))) != 0) break;
    }
  }
  for (; i < T; ++i) acc[0] = __fadd_rn(acc[0], term(i));
  for (int j = 1; j < 4; ++j) acc[0] = __fadd_rn(acc[0], acc[j]);
  return dev_round_to(__fdiv_rn(acc[0], (float)T), dt);
}

// mode kKeyAll: scores, selection on one lane, codes (small pages).
// mode kKeyScores: scores only, written as D floats at the start of the
//   page's low-code region (overwritten later by kKeyCodes).
// mode kKeyCodes: codes with the promoted channels read back from `idx`.
constexpr int kKeyAll = 0, kKeyScores = 1, kKeyCodes = 2;

__global__ void __launch_bounds__(kThreads) quantize_key_pages_tiled(KeyParams k, int mode) {
  extern __shared__ __attribute__((aligned(16))) uint8_t ksm[];
  const dkv_key_pages_args& a = k.a;
  const int bh = blockIdx.x, page = blockIdx.y;
  const int b = bh / (int)a.H, h = bh % (int)a.H;
  const int D = (int)a.D, T = (int)a.page_tokens, dt = (int)a.src_dtype, meta = (int)a.meta_dtype;
  const bool mixed = a.key_mode == DKV_KEY_MIXED;
  const int K = mixed ? (int)a.promoted : 0;
  const int G = (int)k.G, group = (int)a.group;
  const int rs = key_tile_row_bytes(D);
  const int bits = mixed ? 2 : (int)a.bits;
  const int per_byte = 8 / bits;
  const int row_bytes = mixed ? G * (int)k.nb : (int)k.pk;  // packed bytes per channel row

  uint8_t* tile = ksm;                                           // [T][rs]
  float* score = (float*)(ksm + ((T * rs + 15) & ~15));          // [D]
  float* mn_s = score + D;                                       // [D][G]
  float* sc_s = mn_s + D * G;                                    // [D][G]
  int32_t* slot = (int32_t*)(sc_s + D * G);                      // [D]
  int32_t* sel = slot + D;                                       // [D]
  SelItem* work = (SelItem*)(sel + D);                           // [D]
  uint8_t* lowb = (uint8_t*)(((uintptr_t)(work + D) + 15) & ~(uintptr_t)15);  // [D][row_bytes]
  uint8_t* highb = lowb + ((D * row_bytes + 15) & ~15);          // [K][row_bytes]

  // ---- stage the tile ----
  const uint16_t* src = (const uint16_t*)a.src + b * a.sb + h * a.sh + (int64_t)page * T * a.st;
  const int vecs = D / 8;
#pragma unroll 8  // lets the loads of several rows issue before their LDS writes
  for (int i = threadIdx.x; i < T * vecs; i += kThreads) {
    const int t = i / vecs, c8 = i % vecs;
    const uint4 w = *(const uint4*)(src + (int64_t)t * a.st + 8 * c8);
    uint32_t* dst = (uint32_t*)(tile + t * rs + 16 * c8);
    dst[0] = w.x;
    dst[1] = w.y;
    dst[2] = w.z;
    dst[3] = w.w;
  }
  for (int c = threadIdx.x; c < D; c += kThreads) slot[c] = -1;
  __syncthreads();

  // ---- per-channel statistics and scores ----
  for (int c = threadIdx.x; c < D; c += kThreads) {
    for (int g = 0; g < G; ++g) {
      float mn = tile_elem(tile, rs, T, g * group, c, dt), mx = mn;
      for (int j = 1; j < group; ++j) {
        const float x = tile_elem(tile, rs, T, g * group + j, c, dt);
        mn = nmin(mn, x);
        mx = nmax(mx, x);
      }
      if (mode != kKeyCodes) flag_nonfinite(a.nonfinite, mn, mx);
      mn_s[c * G + g] = mn;
      sc_s[c * G + g] = mx;  // max for now; the scale needs qmax, known after selection
    }
    if (mode != kKeyCodes && mixed && K > 0 && K < D && a.selection != DKV_SELECT_GIVEN) {
      float sc;
      if (a.selection == DKV_SELECT_MAGNITUDE) {
        sc = tile_channel_mean(tile, rs, T, c, dt, 0, 0.f);
      } else {
        const float m = tile_channel_mean(tile, rs, T, c, dt, 2, 0.f);  // mixed.py:159-160
        sc = tile_channel_mean(tile, rs, T, c, dt, 1, m);
      }
      if (mode == kKeyScores)
        ((float*)(a.low + page * a.low_page_stride + (int64_t)bh * D * row_bytes))[c] = sc;
      else
        score[c] = sc;
    }
  }
  if (mode == kKeyScores) return;
  __syncthreads();

  // ---- channel selection ----
  if (mixed && K > 0) {
    const int32_t* idx_in = (const int32_t*)((const char*)a.idx + page * a.idx_page_stride) + (int64_t)bh * K;
    if (K < D && a.selection != DKV_SELECT_GIVEN) {
      if (mode == kKeyCodes) {
        for (int j = threadIdx.x; j < K; j += kThreads) sel[j] = idx_in[j];
      } else if (threadIdx.x == 0) {
        select_topk(score, D, K, work, sel);
      }
    } else {
      for (int j = threadIdx.x; j < K; j += kThreads) sel[j] = (K == D) ? j : a.given_idx[h * K + j];
    }
    __syncthreads();
    for (int j = threadIdx.x; j < K; j += kThreads) {
      const int32_t ch = sel[j];
      if (ch >= 0 && ch < D) slot[ch] = j;
    }
    int32_t* idx_out = (int32_t*)((char*)a.idx + page * a.idx_page_stride) + (int64_t)bh * K;
    for (int j = threadIdx.x; j < K; j += kThreads) idx_out[j] = sel[j];
    __syncthreads();
  }

  // ---- scales and zero points ----
  void* scale = (char*)a.scale + page * a.scale_page_stride;
  void* zero = (char*)a.zero + page * a.zero_page_stride;
  for (int i = threadIdx.x; i < D * G; i += kThreads) {
    const int c = i / G;
    const float qmax = mixed ? (slot[c] >= 0 ? 15.0f : 3.0f) : (float)((1 << a.bits) - 1);
    const float mn = mn_s[i];
    const float sc = dev_group_scale(mn, sc_s[i], qmax, dt);
    sc_s[i] = sc;
    dev_store_meta(scale, (int64_t)bh * D * G + i, sc, meta);
    dev_store_meta(zero, (int64_t)bh * D * G + i, mn, meta);
  }
  __syncthreads();

  // ---- codes: thread (channel c, byte p), channel fastest ----
  for (int i = threadIdx.x; i < D * row_bytes; i += kThreads) {
    const int c = i % D, p = i / D;
    const int32_t sl = mixed ? slot[c] : -1;
    const float qmax = mixed ? (sl >= 0 ? 15.0f : 3.0f) : (float)((1 << a.bits) - 1);
    uint32_t lo = 0, hi = 0;
    if (mixed) {
      // byte p of a channel row: group p / nb, tokens 4 (p % nb) + j of that group
      const int g = p / (int)k.nb, q = p % (int)k.nb;
      const float mn = mn_s[c * G + g], sc = sc_s[c * G + g];
      for (int j = 0; j < 4; ++j) {
        const int w = 4 * q + j;
        if (w >= group) break;
        const uint32_t code = dev_group_code(tile_elem(tile, rs, T, g * group + w, c, dt), mn, sc, qmax, dt);
        lo |= (code & 3u) << (2 * j);
        hi |= (code >> 2) << (2 * j);
      }
      if (sl >= 0) highb[sl * row_bytes + p] = (uint8_t)hi;
    } else {
      const int padded = G * group;
      for (int j = 0; j < per_byte; ++j) {
        const int t = p * per_byte + j;
        if (t >= padded) break;
        const int g = t / group;
        lo |= dev_group_code(tile_elem(tile, rs, T, t, c, dt), mn_s[c * G + g], sc_s[c * G + g], qmax, dt)
              << (j * bits);
      }
    }
    lowb[c * row_bytes + p] = (uint8_t)lo;
  }
  __syncthreads();

  // ---- write the packed rows (contiguous per (batch, head)) ----
  uint8_t* low = a.low + page * a.low_page_stride + (int64_t)bh * D * row_bytes;
  const int lbytes = D * row_bytes;
  for (int i = threadIdx.x; i < lbytes / 16; i += kThreads) ((uint4*)low)[i] = ((const uint4*)lowb)[i];
  for (int i = (lbytes / 16) * 16 + threadIdx.x; i < lbytes; i += kThreads) low[i] = lowb[i];
  if (mixed && K > 0) {
    uint8_t* high = a.high + page * a.high_page_stride + (int64_t)bh * K * row_bytes;
    const int hbytes = K * row_bytes;
    for (int i = threadIdx.x; i < hbytes / 16; i += kThreads) ((uint4*)high)[i] = ((const uint4*)highb)[i];
    for (int i = (hbytes / 16) * 16 + threadIdx.x; i < hbytes; i += kThreads) high[i] = highb[i];
  }
}

// Single-pass key page kernel for the common shape: head_dim 128, at most 128
// tokens per page, one key group per page, 16-bit source with unit channel
// stride.  One workgroup per (batch * head, page), 256 threads:
//   1. the page's [T][128] tile is staged in LDS with 16-byte loads;
//   2. thread (channel c, half h) sums its channel's 16-token chunks of the
//      half sequentially (and takes min / max); one thread per channel then
//      adds the chunk sums in ATen's cascade order, so the mean is bit for bit
//      the serial cascade's (channel_mean);
//   3. selection: each channel's rank is the number of channels with a larger
//      score; with all scores distinct, rank < K is the promoted set in
//      torch.topk(sorted=True) order.  A page with equal (or NaN) scores needs
//      the exact libstdc++ order, which wave 0 computes (wave_select_topk)
//      while the other waves wait.  Equal bf16 scores are the rule, not the
//      exception (32 of 128 means in about one binade), so for many pages the
//      launcher runs mode kKeyScores (steps 1-2, scores to the page's low-code
//      region), key_select_pages (one wave per page: many selections in
//      flight hide the latency of their dependent LDS steps, which a
//      workgroup waiting on its own cannot) and mode kKeyCodes (steps 1, 4, 5
//      with the channels and the channel ranges read back); mode kKeyAll does
//      everything here (pages without a data-dependent selection, and few
//      pages);
//   4. scales, zero points and one reciprocal per channel;
//   5. codes: thread (c, half) quantizes 64 tokens of channel c with the
//      exact chain (div_rn); the packed rows leave through LDS.
constexpr int kFastKeyD = 128, kFastKeyT = 128;

template <int SRC>
__device__ __forceinline__ float tile_x(const uint16_t* tile, int t, int c) {
  const uint16_t bits = tile[t * kFastKeyD + c];
  return SRC == kBF16 ? bf16_to_f32(bits) : (float)__builtin_bit_cast(_Float16, bits);
}

// Sum of f(x) over the 16 tokens tb .. tb + 15 of channel c, sequentially
// (tokens at or past T add an exact zero).  The 16 reads are issued before
// the first add.  mode 0: |x|; 1: rnd(rnd(x - m)^2); 2: x.  Also folds the
// tokens into mn / mx when MINMAX (tokens past T repeat the last one, which
// leaves min and max unchanged).  FULL: T is the full page (no clamping, and
// the reads take constant offsets from one address).
template <int SRC, bool MINMAX, bool FULL>
__device__ __forceinline__ float key_chunk_sum(const uint16_t* tile, int c, int tb, int T, int mode, float m,
                                               float& mn, float& mx) {
  float xs[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) xs[j] = tile_x<SRC>(tile, FULL ? tb + j : min(tb + j, T - 1), c);
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const float x = xs[j];
    if (MINMAX) {
      mn = nmin(mn, x);
      mx = nmax(mx, x);
    }
    float term = x;
    if (mode == 0) term = fabsf(x);
    if (mode == 1) {
      const float d = src_round<SRC>(x - m);
      term = src_round<SRC>(d * d);
    }
    acc = acc + ((FULL || tb + j < T) ? term : 0.f);
  }
  return acc;
}

// The cascade of channel_mean (level power 4: 16-term chunks, level-1
// partials summed in order; pages of at most 128 tokens never reach level 2)
// over the chunk sums csum[k][c], then one division and the rounding to the
// source dtype.  A short last chunk is the cascade's remainder, added first.
template <int SRC>
__device__ __forceinline__ float key_cascade_mean(const float* csum, int c, int T) {
  const int full = T >> 4;
  float acc1 = 0.f;
  for (int k = 0; k < full; ++k) acc1 = acc1 + csum[k * kFastKeyD + c];
  float acc0 = (T & 15) ? csum[full * kFastKeyD + c] : 0.f;
  acc0 = acc0 + acc1;
  acc0 = acc0 + 0.f;  // levels 2 and 3 hold zero
  acc0 = acc0 + 0.f;
  return src_round<SRC>(__fdiv_rn(acc0, (float)T));
}

// BITS: code width of the low codes (2 for mixed keys, else the uniform width).
// FULL: every page holds kFastKeyT tokens (token indices need no clamping,
// and the tile reads take constant offsets: about 3 VALU less per read).
template <int SRC, int BITS, bool FULL>
__global__ void __launch_bounds__(kThreads) quantize_key_pages_fast(KeyParams k, int mode) {
  __shared__ __attribute__((aligned(16))) uint16_t tile[kFastKeyT * kFastKeyD];
  __shared__ float csum[8 * kFastKeyD];
  __shared__ float part_mn[2][kFastKeyD], part_mx[2][kFastKeyD];
  __shared__ __attribute__((aligned(16))) float score[kFastKeyD];
  __shared__ float ch_mn[kFastKeyD], ch_s[kFastKeyD], ch_y[kFastKeyD];
  __shared__ int32_t slot[kFastKeyD], sel[kFastKeyD];
  __shared__ uint32_t sel_words[kFastKeyD];
  __shared__ uint8_t sel_lpos[kFastKeyD], sel_rpos[kFastKeyD];
  __shared__ int sel_stack[3 * kSelectStack];
  const dkv_key_pages_args& a = k.a;
  const int bh = blockIdx.x, page = blockIdx.y;
  const int b = bh / (int)a.H, h = bh % (int)a.H;
  const int T = FULL ? kFastKeyT : (int)a.page_tokens, meta = (int)a.meta_dtype;
  const bool mixed = a.key_mode == DKV_KEY_MIXED;
  const int K = mixed ? (int)a.promoted : 0;
  constexpr int row_bytes = kFastKeyT * BITS / 8;  // one group of up to 128 tokens per channel row
  const int tid = threadIdx.x;

  // ---- 1. stage the tile: every load is issued before the first LDS write
  // (a loop that stored each load before issuing the next waited one memory
  // round trip per row group) ----
  const uint16_t* src = (const uint16_t*)a.src + b * a.sb + h * a.sh + (int64_t)page * T * a.st;
  {
    constexpr int kSteps = kFastKeyT * (kFastKeyD / 8) / kThreads;  // 8
    uint4 w[kSteps];
#pragma unroll
    for (int j = 0; j < kSteps; ++j) {
      const int i = tid + j * kThreads, t = FULL ? i >> 4 : min(i >> 4, T - 1), c8 = i & 15;
      w[j] = *(const uint4*)(src + (int64_t)t * a.st + 8 * c8);
    }
    // rows past T hold copies of row T - 1 (reads clamp to T - 1 anyway); an
    // unconditional store keeps the compiler from sinking each load into a
    // branch next to its store
#pragma unroll
    for (int j = 0; j < kSteps; ++j) {
      const int i = tid + j * kThreads;
      *(uint4*)(tile + (i >> 4) * kFastKeyD + 8 * (i & 15)) = w[j];
    }
  }
  if (tid < kFastKeyD) slot[tid] = -1;
  __syncthreads();

  // ---- 2. statistics: thread (channel c, half) covers tokens 64 half .. 64 half + 63 ----
  const int c = tid & (kFastKeyD - 1), half = tid >> 7;
  const bool select = mixed && K > 0 && K < kFastKeyD && a.selection != DKV_SELECT_GIVEN && mode != kKeyCodes;
  const bool magnitude = a.selection == DKV_SELECT_MAGNITUDE;
  if (mode != kKeyCodes) {  // the codes pass reads the channel min / max its scores pass stored
    float mn = INFINITY, mx = -INFINITY;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int tb = 64 * half + 16 * q;
      if (tb < T) {
        const float sum = key_chunk_sum<SRC, true, FULL>(tile, c, tb, T, magnitude ? 0 : 2, 0.f, mn, mx);
        if (select) csum[(tb >> 4) * kFastKeyD + c] = sum;
      }
    }
    part_mn[half][c] = mn;
    part_mx[half][c] = mx;
  }
  if (select) {
    __syncthreads();
    if (half == 0) score[c] = key_cascade_mean<SRC>(csum, c, T);  // magnitude score, or the variance's mean
    if (!magnitude) {  // variance (mixed.py:158-162): mean squared deviation from that mean
      __syncthreads();
      const float m = score[c];
      float mn = 0.f, mx = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int tb = 64 * half + 16 * q;
        if (tb < T) csum[(tb >> 4) * kFastKeyD + c] = key_chunk_sum<SRC, false, FULL>(tile, c, tb, T, 1, m, mn, mx);
      }
      __syncthreads();
      if (half == 0) score[c] = key_cascade_mean<SRC>(csum, c, T);
    }
  }
  __syncthreads();
  // kKeyScores leaves [score | min | max] x 128 floats at the start of the
  // page's low-code region (1.5 KiB of its 128 x row_bytes); kKeyCodes reads
  // min and max back and overwrites the region with the codes
  static_assert(3 * kFastKeyD * 4 <= kFastKeyD * row_bytes, "scores and ranges must fit the low-code region");
  float* stash = (float*)(a.low + page * a.low_page_stride + (int64_t)bh * kFastKeyD * row_bytes);
  if (mode == kKeyScores) {
    if (half == 0) {
      const float mn = nmin(part_mn[0][c], part_mn[1][c]), mx = nmax(part_mx[0][c], part_mx[1][c]);
      stash[c] = score[c];
      stash[kFastKeyD + c] = mn;
      stash[2 * kFastKeyD + c] = mx;
      flag_nonfinite(a.nonfinite, mn, mx);
    }
    return;
  }
  if (half == 0) {
    if (mode == kKeyCodes) {
      ch_mn[c] = stash[kFastKeyD + c];
      ch_s[c] = stash[2 * kFastKeyD + c];  // max for now
    } else {
      ch_mn[c] = nmin(part_mn[0][c], part_mn[1][c]);
      ch_s[c] = nmax(part_mx[0][c], part_mx[1][c]);  // max for now
      flag_nonfinite(a.nonfinite, ch_mn[c], ch_s[c]);
    }
  }

  // ---- 3. channel selection ----
  if (mixed && K > 0) {
    if (mode == kKeyCodes && K < kFastKeyD && a.selection != DKV_SELECT_GIVEN) {
      if (tid < K) sel[tid] = ((const int32_t*)((const char*)a.idx + page * a.idx_page_stride))[(int64_t)bh * K + tid];
    } else if (select) {
      bool tie = false;
      int rank = 0;
      if (half == 0) {
        const float v = score[c];
        tie = v != v;
#pragma unroll 8
        for (int j = 0; j < kFastKeyD; j += 4) {
          const float4 u = *(const float4*)(score + j);
          rank += (u.x > v) + (u.y > v) + (u.z > v) + (u.w > v);
          tie |= ((u.x == v) & (j != c)) | ((u.y == v) & (j + 1 != c)) | ((u.z == v) & (j + 2 != c)) |
                 ((u.w == v) & (j + 3 != c));
        }
      }
      if (__syncthreads_or(tie)) {
        if (tid < 64)
          wave_select_topk(score, kFastKeyD, K, tid, WaveSelBuffers{sel_words, sel_lpos, sel_rpos, sel_stack}, sel);
      } else if (half == 0 && rank < K) {
        sel[rank] = c;
      }
    } else if (tid < K) {
      sel[tid] = (K == kFastKeyD) ? tid : a.given_idx[h * K + tid];
    }
    __syncthreads();
    int32_t* idx_out = (int32_t*)((char*)a.idx + page * a.idx_page_stride) + (int64_t)bh * K;
    if (tid < K) {
      const int32_t ch = sel[tid];
      if (ch >= 0 && ch < kFastKeyD) slot[ch] = tid;
      idx_out[tid] = ch;
    }
  }
  __syncthreads();

  // ---- 4. scales and zero points (one group per channel) ----
  if (half == 0) {
    const float qmax = mixed ? (slot[c] >= 0 ? 15.0f : 3.0f) : (float)((1 << BITS) - 1);
    const float mn = ch_mn[c];
    const float s = dev_group_scale(mn, ch_s[c], qmax, SRC);
    ch_s[c] = s;
    ch_y[c] = __fdiv_rn(1.0f, s);
    void* scale = (char*)a.scale + page * a.scale_page_stride;
    void* zero = (char*)a.zero + page * a.zero_page_stride;
    dev_store_meta(scale, (int64_t)bh * kFastKeyD + c, s, meta);
    dev_store_meta(zero, (int64_t)bh * kFastKeyD + c, mn, meta);
  }
  __syncthreads();

  // ---- 5. codes: thread (c, half) packs row bytes half * row_bytes / 2 ..
  // of channel c into registers; once every tile read is done the packed rows
  // go through the tile's LDS (rows kCodePitch bytes apart, so the lanes'
  // 16-byte writes fall in different banks) and leave in 16-byte stores of
  // consecutive addresses ----
  {
    constexpr int per_byte = 8 / BITS, tpd = 4 * per_byte;  // tokens per code dword
    constexpr int bpp = row_bytes / 2, nw = bpp / 4;        // bytes and dwords per thread
    constexpr int kCodePitch = row_bytes + 16;
    static_assert(kFastKeyD * (BITS == 2 ? 2 : 1) * kCodePitch <= (int)sizeof(tile), "packed rows must fit the tile");
    const int sl = slot[c];
    const float mn = ch_mn[c], s = ch_s[c], y = ch_y[c];
    uint32_t lo[nw], hi[nw];
#pragma unroll
    for (int w = 0; w < nw; ++w) {
      const int tb = (half * bpp + 4 * w) * per_byte;
      float xs[tpd];
#pragma unroll
      for (int j = 0; j < tpd; ++j)
        xs[j] = tile_x<SRC>(tile, FULL ? tb + j : min(tb + j, T - 1), c);  // padding repeats the last token
      hi[w] = 0;
      // four tokens' codes at a time, each conversion writing its code at its
      // byte of the packed layout (qmax is 3 or 15 here, or the byte range
      // for 8-bit keys), then the fields combined
      if (BITS == 8) {
        float q[4];
        chain_quotients4<SRC>(xs, mn, s, y, q);
        lo[w] = codes_as_bytes(q);
      } else if (BITS == 4) {
        uint32_t plane[2] = {0u, 0u};
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          float q[4];
          chain_quotients4<SRC>(&xs[4 * g], mn, s, y, q);
          codes_to_planes4(q, g, plane);
        }
        lo[w] = pack4(plane);
      } else {
        uint32_t plane[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          float q[4];
          chain_quotients4<SRC>(&xs[4 * g], mn, s, y, q);
          codes_to_planes2(q, g, plane);
        }
        if (mixed) {  // codes up to 15: low and high two bits
          lo[w] = pack2_low(plane);
          hi[w] = pack2_high(plane);
        } else {
          lo[w] = pack2(plane);
        }
      }
    }
    __syncthreads();  // the tile is read for the last time above
    uint8_t* lowb = (uint8_t*)tile;                      // [128][kCodePitch]: low codes
    uint8_t* highb = lowb + kFastKeyD * kCodePitch;      // [K][kCodePitch]: high codes of the promoted slots
#pragma unroll
    for (int w = 0; w < nw; w += 4) {
      *(uint4*)(lowb + c * kCodePitch + half * bpp + 4 * w) = make_uint4(lo[w], lo[w + 1], lo[w + 2], lo[w + 3]);
      if (mixed && sl >= 0)
        *(uint4*)(highb + sl * kCodePitch + half * bpp + 4 * w) = make_uint4(hi[w], hi[w + 1], hi[w + 2], hi[w + 3]);
    }
    __syncthreads();
    constexpr int q_row = row_bytes / 16;  // 16-byte pieces per packed row
    uint4* low = (uint4*)(a.low + page * a.low_page_stride + (int64_t)bh * kFastKeyD * row_bytes);
    for (int i = tid; i < kFastKeyD * q_row; i += kThreads)
      low[i] = *(const uint4*)(lowb + (i / q_row) * kCodePitch + 16 * (i % q_row));
    if (mixed && K > 0) {
      uint4* high = (uint4*)(a.high + page * a.high_page_stride + (int64_t)bh * K * row_bytes);
      for (int i = tid; i < K * q_row; i += kThreads)
        high[i] = *(const uint4*)(highb + (i / q_row) * kCodePitch + 16 * (i % q_row));
    }
  }
}

// Promoted-channel selection for many pages at once: one wave per
// (batch * head, page) runs the exact top-k (wave_select_topk) on the scores
// kKeyScores left in the page's low-code region and writes the channel
// indices.  The selection is a chain of dependent LDS steps; its small LDS
// footprint lets many such waves run side by side and hide that latency.
constexpr int kSelectMaxD = 128;

struct SelectLds {
  float sc[kSelectMaxD];
  uint32_t words[kSelectMaxD];
  uint8_t lpos[kSelectMaxD], rpos[kSelectMaxD];
  int stack[3 * kSelectStack];
};

__device__ __forceinline__ void select_page(const KeyParams& k, int row_bytes, int64_t item, int lane, SelectLds& l) {
  const dkv_key_pages_args& a = k.a;
  const int64_t bhs = a.B * a.H;
  const int64_t page = item / bhs, bh = item % bhs;
  const int D = (int)a.D, K = (int)a.promoted;
  const float* score = (const float*)(a.low + page * a.low_page_stride + bh * D * row_bytes);
  for (int j = lane; j < D; j += 64) l.sc[j] = score[j];
  DeviceWave{lane}.sync();
  int32_t* idx_out = (int32_t*)((char*)a.idx + page * a.idx_page_stride) + bh * K;
  wave_select_topk(l.sc, D, K, lane, WaveSelBuffers{l.words, l.lpos, l.rpos, l.stack}, idx_out);
}

__global__ void __launch_bounds__(64) key_select_pages(KeyParams k, int row_bytes) {
  __shared__ SelectLds l;
  select_page(k, row_bytes, blockIdx.x, threadIdx.x, l);
}

// The key path's channel selection and a value-row job in one launch.
// The first workgroups make the call's dense token copies
// (kCopyUnitsPerThread units per thread), the next sel_blocks select (one
// wave per page, as key_select_pages) and the last gx * gy quantize value rows
// (the gx x gy grid of quantize_rows_vec).  A selection wave mostly waits on
// its LDS steps; the copies and the value rows use each SIMD meanwhile.
// (Spreading the selection workgroups among the value rows' was slower: a
// selection wave's chain of dependent steps stretches when VALU-bound row
// waves share its SIMD.)
constexpr int kSelectWaves = kThreads / 64;
constexpr int kCopyUnitsPerThread = 4;

__global__ void __launch_bounds__(kThreads) copy_token_blocks_kernel(dkv::CopyParams cp) {
  const int64_t u = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (u < cp.first[cp.n]) dkv::copy_token_unit(cp, u);
}

__host__ inline int64_t copy_blocks_for(const dkv::CopyParams& cp) {
  const int64_t per_block = (int64_t)kThreads * kCopyUnitsPerThread;
  return (cp.first[cp.n] + per_block - 1) / per_block;
}
// Shared launches pay off while every selection wave is resident at once (one
// wave per page, 256 CUs x 32 waves); past that the selections queue in rounds
// and the value rows wait behind them, so the two run as separate launches.
constexpr int64_t kSelectFuseMaxPages = 8192;

template <int BITS, int SRC, int E>
__global__ void __launch_bounds__(kThreads) select_pages_and_rows(KeyParams k, int row_bytes, int64_t items,
                                                                  int64_t sel_blocks, RowsParams p, int lpg,
                                                                  int row_shift, int64_t gx, int64_t gy,
                                                                  dkv::CopyParams cp, int64_t copy_blocks) {
  __shared__ SelectLds l[kSelectWaves];
  if ((int64_t)blockIdx.x < copy_blocks) {
    const int64_t u0 = (int64_t)blockIdx.x * kThreads * kCopyUnitsPerThread + threadIdx.x;
    const int64_t units = cp.first[cp.n];
#pragma unroll
    for (int i = 0; i < kCopyUnitsPerThread; ++i) {
      const int64_t u = u0 + (int64_t)i * kThreads;
      if (u < units) dkv::copy_token_unit(cp, u);
    }
    return;
  }
  const int64_t sb = (int64_t)blockIdx.x - copy_blocks;
  if (sb < sel_blocks) {
    const int wave = threadIdx.x >> 6;
    const int64_t item = sb * kSelectWaves + wave;
    if (item < items) select_page(k, row_bytes, item, threadIdx.x & 63, l[wave]);
    return;
  }
  const int64_t b = sb - sel_blocks;
  rows_vec_body<BITS, SRC, E>(p, lpg, row_shift, b % gx, b / gx, gx, gy);
}

__host__ inline size_t key_tiled_smem(int D, int T, int G, int K, int row_bytes) {
  size_t o = ((size_t)T * key_tile_row_bytes(D) + 15) & ~(size_t)15;
  o += sizeof(float) * ((size_t)D + 2 * (size_t)D * G) + 2 * sizeof(int32_t) * D + sizeof(SelItem) * D;
  o = (o + 15) & ~(size_t)15;
  o += ((size_t)D * row_bytes + 15) & ~(size_t)15;
  o += (size_t)K * row_bytes;
  return o;
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
  dev_dequant_store(out, r * out_stride + i, code, dev_load_meta(scale, r * groups + g, meta),
                    dev_load_meta(zero, r * groups + g, meta), meta, out_dt);
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
  dev_dequant_store(out, (bh * T + t) * D + c, code, dev_load_meta(scale, mi, meta), dev_load_meta(zero, mi, meta),
                    meta, out_dt);
}

bool valid_float_dtype(int64_t dt) { return dt == kF32 || dt == kF16 || dt == kBF16 || dt == kF64; }
bool valid_meta_dtype(int64_t dt) { return dt == kF32 || dt == kF16 || dt == kBF16 || dt == kF64; }
bool valid_bits(int64_t b) { return b == 2 || b == 4 || b == 8; }

}  // namespace

// A planned value-row launch: parameters, kernel choice and grid.
struct RowsLaunch {
  RowsParams p;
  int64_t rows;
  bool vec;                // quantize_rows_vec applies
  int epl;                 // its elements per lane (8 or 16)
  int lpg, row_shift;      // its lanes per group and log2(lanes per row) (-1: not a power of two)
  int64_t gx, gy;          // its grid
  int bits, src_dtype;
};

// Validate a value-row job and plan its launch (nothing is launched).
static int prepare_rows(const void* src, int src_dtype, int64_t blocks, int64_t block_stride, int64_t block_rows,
                        int64_t n, int64_t row_stride, int64_t elem_stride, int bits, int64_t group, uint8_t* values,
                        void* scale, void* zero, int meta_dtype, uint32_t* nonfinite, int64_t out_block_rows,
                        int64_t out_row0, RowsLaunch& L) {
  const int64_t rows = blocks * block_rows;
  DKV_CHECK(valid_float_dtype(src_dtype), DKV_ERR_DTYPE, "quantize expects a floating-point tensor (f64/f32/f16/bf16)");
  DKV_CHECK(valid_meta_dtype(meta_dtype), DKV_ERR_DTYPE, "metadata dtype must be floating point");
  DKV_CHECK(valid_bits(bits), DKV_ERR_INVALID, "bits must be one of (2, 4, 8), got %d", bits);
  DKV_CHECK(group > 0, DKV_ERR_INVALID, "group_size must be a positive integer, got %lld", (long long)group);
  DKV_CHECK(n > 0 && rows >= 0, DKV_ERR_INVALID, "quantize does not support an empty final dimension");
  RowsParams& p = L.p;
  p.src = src;
  p.rows = rows;
  p.blocks = blocks;
  p.block_rows = block_rows;
  p.block_stride = block_stride;
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
  p.nonfinite = nonfinite;
  p.out_block_rows = out_block_rows > 0 ? out_block_rows : block_rows;
  p.out_row0 = out_row0;
  DKV_CHECK(p.out_block_rows >= block_rows && out_row0 >= 0 && out_row0 <= p.out_block_rows - block_rows,
            DKV_ERR_INVALID, "value rows: output rows [out_row0, out_row0 + block_rows) must lie in out_block_rows");
  L.rows = rows;
  L.bits = bits;
  L.src_dtype = src_dtype;
  const int esize = src_dtype == kF64 ? 8 : src_dtype == kF32 ? 4 : 2;
  L.vec = elem_stride == 1 && n % 8 == 0 && group % 8 == 0 && group <= 512 && (group & (group - 1)) == 0 &&
          n % group == 0 && ((uintptr_t)src % 16) == 0 && (row_stride * esize) % 16 == 0 &&
          (block_stride * esize) % 16 == 0 &&
          (src_dtype == kF32 || src_dtype == kF16 || src_dtype == kBF16) && ((uintptr_t)values % 8) == 0 &&
          (p.packed_bytes * bits) % 8 == 0 && (p.packed_bytes % 8) == 0;
  // 16 elements per lane where groups and rows split into 16s and each lane's
  // 2 * bits bytes of codes are aligned for one store
  L.epl = (group % 16 == 0 && n % 16 == 0 && ((uintptr_t)values % (2 * bits)) == 0) ? 16 : 8;
  L.lpg = (int)(group / L.epl);
  const int64_t lpr = n / L.epl;
  L.row_shift = (lpr & (lpr - 1)) == 0 ? __builtin_ctzll((unsigned long long)lpr) : -1;
  // x: workgroups over one block's lanes; y: row blocks (the kernel strides
  // over both, so the grid is capped at about 2^20 workgroups)
  const int64_t lanes = block_rows * lpr;
  L.gy = std::max<int64_t>(std::min<int64_t>(blocks, 65535), 1);
  L.gx = std::max<int64_t>(
      std::min<int64_t>((lanes + kThreads * kRowChunks - 1) / (kThreads * kRowChunks), (1 << 20) / L.gy), 1);
  return DKV_OK;
}

static void launch_rows(const RowsLaunch& L, hipStream_t s) {
  if (L.rows == 0) return;
  const RowsParams& p = L.p;
  if (L.vec) {
#define DKV_ROWS_LAUNCH(B, T)                                                                                      \
  do {                                                                                                             \
    if (L.epl == 16)                                                                                               \
      hipLaunchKernelGGL((quantize_rows_vec<B, T, 16>), dim3((unsigned)L.gx, (unsigned)L.gy), dim3(kThreads), 0, s, \
                         p, L.lpg, L.row_shift);                                                                   \
    else                                                                                                           \
      hipLaunchKernelGGL((quantize_rows_vec<B, T, 8>), dim3((unsigned)L.gx, (unsigned)L.gy), dim3(kThreads), 0, s,  \
                         p, L.lpg, L.row_shift);                                                                   \
  } while (0)
#define DKV_ROWS_BITS(T)                    \
  do {                                      \
    if (L.bits == 2) DKV_ROWS_LAUNCH(2, T);   \
    else if (L.bits == 4) DKV_ROWS_LAUNCH(4, T); \
    else DKV_ROWS_LAUNCH(8, T);             \
  } while (0)
    if (L.src_dtype == kBF16) DKV_ROWS_BITS(kBF16);
    else if (L.src_dtype == kF16) DKV_ROWS_BITS(kF16);
    else DKV_ROWS_BITS(kF32);
#undef DKV_ROWS_BITS
#undef DKV_ROWS_LAUNCH
  } else if (p.group % p.per_byte == 0) {
    const int64_t items = L.rows * p.groups;
    const dim3 grid((unsigned)((items + kThreads - 1) / kThreads));
    if (L.src_dtype == kF64) {
      hipLaunchKernelGGL(quantize_rows_aligned<double>, grid, dim3(kThreads), 0, s, p);
    } else {
      hipLaunchKernelGGL(quantize_rows_aligned<float>, grid, dim3(kThreads), 0, s, p);
    }
  } else {
    const dim3 grid((unsigned)((L.rows + kThreads - 1) / kThreads));
    if (L.src_dtype == kF64) {
      hipLaunchKernelGGL(quantize_rows_serial<double>, grid, dim3(kThreads), 0, s, p);
    } else {
      hipLaunchKernelGGL(quantize_rows_serial<float>, grid, dim3(kThreads), 0, s, p);
    }
  }
}

static int quantize_rows_impl(const void* src, int src_dtype, int64_t blocks, int64_t block_stride,
                              int64_t block_rows, int64_t n, int64_t row_stride, int64_t elem_stride, int bits,
                              int64_t group, uint8_t* values, void* scale, void* zero, int meta_dtype,
                              uint32_t* nonfinite, int64_t out_block_rows, int64_t out_row0, void* stream,
                              const char* name) {
  RowsLaunch L;
  const int rc = prepare_rows(src, src_dtype, blocks, block_stride, block_rows, n, row_stride, elem_stride, bits,
                              group, values, scale, zero, meta_dtype, nonfinite, out_block_rows, out_row0, L);
  if (rc != DKV_OK) return rc;
  if (L.rows == 0) return DKV_OK;
  launch_rows(L, (hipStream_t)stream);
  return dkv_check_launch(name);
}

extern "C" int dkv_quantize_rows(const void* src, int src_dtype, int64_t rows, int64_t n, int64_t row_stride,
                                 int64_t elem_stride, int bits, int64_t group, uint8_t* values, void* scale,
                                 void* zero, int meta_dtype, void* stream) {
  DKV_CHECK(rows >= 0, DKV_ERR_INVALID, "rows must be non-negative");
  return quantize_rows_impl(src, src_dtype, 1, 0, rows, n, row_stride, elem_stride, bits, group, values, scale, zero,
                            meta_dtype, nullptr, 0, 0, stream, "dkv_quantize_rows");
}

extern "C" int dkv_quantize_row_blocks(const void* src, int src_dtype, int64_t blocks, int64_t block_stride,
                                       int64_t block_rows, int64_t n, int64_t row_stride, int bits, int64_t group,
                                       uint8_t* values, void* scale, void* zero, int meta_dtype, void* stream) {
  DKV_CHECK(blocks >= 0 && block_rows >= 0, DKV_ERR_INVALID, "blocks and block_rows must be non-negative");
  DKV_CHECK(block_rows == 0 || blocks <= INT64_MAX / block_rows, DKV_ERR_INVALID, "blocks * block_rows overflows");
  return quantize_rows_impl(src, src_dtype, blocks, block_stride, block_rows, n, row_stride, 1, bits, group, values,
                            scale, zero, meta_dtype, nullptr, 0, 0, stream, "dkv_quantize_row_blocks");
}

extern "C" int dkv_quantize_value_rows(const dkv_value_rows_args* args, void* stream) {
  DKV_CHECK(args != nullptr, DKV_ERR_INVALID, "args is NULL");
  const dkv_value_rows_args& v = *args;
  DKV_CHECK(v.blocks >= 0 && v.block_rows >= 0, DKV_ERR_INVALID, "blocks and block_rows must be non-negative");
  DKV_CHECK(v.block_rows == 0 || v.blocks <= INT64_MAX / v.block_rows, DKV_ERR_INVALID, "blocks * block_rows overflows");
  return quantize_rows_impl(v.src, (int)v.src_dtype, v.blocks, v.block_stride, v.block_rows, v.n, v.row_stride, 1,
                            (int)v.bits, v.group, v.values, v.scale, v.zero, (int)v.meta_dtype, v.nonfinite,
                            v.out_block_rows, v.out_row0, stream, "dkv_quantize_value_rows");
}

extern "C" int dkv_quantize_key_pages(const dkv_key_pages_args* args, void* stream) {
  DKV_CHECK(args != nullptr, DKV_ERR_INVALID, "args is NULL");
  const dkv_key_pages_args& a = *args;
  DKV_CHECK(valid_float_dtype(a.src_dtype), DKV_ERR_DTYPE, "key_states must be floating point (f64/f32/f16/bf16)");
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
  DKV_CHECK(a.B * a.H * a.n_pages <= 0x7fffffffLL, DKV_ERR_UNSUPPORTED, "too many pages for one launch");
  // the optional value rows: validated and planned before anything launches
  RowsLaunch VL;
  const bool with_values = a.values != nullptr;
  bool values_done = false;
  if (with_values) {
    const dkv_value_rows_args& v = *a.values;
    DKV_CHECK(v.blocks >= 0 && v.block_rows >= 0, DKV_ERR_INVALID, "value blocks and block_rows must be non-negative");
    DKV_CHECK(v.block_rows == 0 || v.blocks <= INT64_MAX / v.block_rows, DKV_ERR_INVALID,
              "value blocks * block_rows overflows");
    const int rc = prepare_rows(v.src, (int)v.src_dtype, v.blocks, v.block_stride, v.block_rows, v.n, v.row_stride, 1,
                                (int)v.bits, v.group, v.values, v.scale, v.zero, (int)v.meta_dtype, v.nonfinite,
                                v.out_block_rows, v.out_row0, VL);
    if (rc != DKV_OK) return rc;
  }
  // the optional dense copies: validated before anything launches; they ride in the
  // selection + value-row launch when it runs, else they get a launch of their own last
  dkv::CopyParams CP;
  {
    const int rc = dkv::prepare_copies(a.copies, a.n_copies, CP, "dkv_quantize_key_pages copies");
    if (rc != DKV_OK) return rc;
  }
  bool copies_done = CP.first[CP.n] == 0;
  hipStream_t s = (hipStream_t)stream;
  auto finish = [&]() {
    if (with_values && !values_done) launch_rows(VL, s);
    if (!copies_done) {
      const int64_t units = CP.first[CP.n];
      hipLaunchKernelGGL(copy_token_blocks_kernel, dim3((unsigned)((units + kThreads - 1) / kThreads)),
                         dim3(kThreads), 0, s, CP);
    }
    return dkv_check_launch("dkv_quantize_key_pages");
  };
  if (a.n_pages == 0) return finish();
  KeyParams k;
  k.a = a;
  k.G = (a.page_tokens + a.group - 1) / a.group;
  k.nb = (a.group + 3) / 4;
  const int per_byte = a.key_mode == DKV_KEY_UNIFORM ? (int)(8 / a.bits) : 4;
  k.pk = (k.G * a.group + per_byte - 1) / per_byte;
  const int row_bytes = a.key_mode == DKV_KEY_MIXED ? (int)(k.G * k.nb) : (int)k.pk;
  const int Kp = a.key_mode == DKV_KEY_MIXED ? (int)a.promoted : 0;
  const size_t tiled = key_tiled_smem((int)a.D, (int)a.page_tokens, (int)k.G, Kp, row_bytes);
  const bool use_tiled = (a.src_dtype == kBF16 || a.src_dtype == kF16) && a.sd == 1 && a.D % 8 == 0 &&
                         a.D <= kThreads && a.st % 8 == 0 && a.sb % 8 == 0 && a.sh % 8 == 0 &&
                         ((uintptr_t)a.src % 16) == 0 && ((a.page_tokens * a.st) % 8) == 0 &&
                         (size_t)a.page_tokens * key_tile_row_bytes((int)a.D) <= (size_t)kKeyTileMaxBytes &&
                         tiled <= 64 * 1024 && ((uintptr_t)a.low % 16) == 0 && (a.low_page_stride % 16) == 0 &&
                         ((int64_t)a.D * row_bytes) % 16 == 0 &&
                         (Kp == 0 || (((uintptr_t)a.high % 16) == 0 && (a.high_page_stride % 16) == 0 &&
                                      ((int64_t)Kp * row_bytes) % 16 == 0));
  // the single-pass kernel: head_dim 128, one group of up to 128 tokens per page
  const int fast_bits = a.key_mode == DKV_KEY_MIXED ? 2 : (int)a.bits;
  const bool use_fast = use_tiled && a.D == kFastKeyD && a.page_tokens <= kFastKeyT && a.group >= kFastKeyT &&
                        a.st % 8 == 0 && row_bytes == kFastKeyT * fast_bits / 8 && ((uintptr_t)a.low % 4) == 0 &&
                        (a.low_page_stride % 4) == 0 && (Kp == 0 || (((uintptr_t)a.high % 4) == 0 &&
                                                                       (a.high_page_stride % 4) == 0));
  if (use_fast) {
    const dim3 grid((unsigned)(a.B * a.H), (unsigned)a.n_pages);
#define DKV_KEYF(T, B, M)                                                                                 \
  do {                                                                                                    \
    if (a.page_tokens == kFastKeyT)                                                                       \
      hipLaunchKernelGGL((quantize_key_pages_fast<T, B, true>), grid, dim3(kThreads), 0, s, k, M);        \
    else                                                                                                  \
      hipLaunchKernelGGL((quantize_key_pages_fast<T, B, false>), grid, dim3(kThreads), 0, s, k, M);       \
  } while (0)
#define DKV_KEYF_BITS(T, M)                   \
  do {                                        \
    if (fast_bits == 2) DKV_KEYF(T, 2, M);    \
    else if (fast_bits == 4) DKV_KEYF(T, 4, M); \
    else DKV_KEYF(T, 8, M);                   \
  } while (0)
#define DKV_KEYF_RUN(M)                                \
  do {                                                 \
    if (a.src_dtype == kBF16) DKV_KEYF_BITS(kBF16, M); \
    else DKV_KEYF_BITS(kF16, M);                       \
  } while (0)
    // a data-dependent selection over more than a few pages: scores, one
    // wave per page selects, codes
    const bool select = a.key_mode == DKV_KEY_MIXED && Kp > 0 && Kp < a.D && a.selection != DKV_SELECT_GIVEN;
    if (select && a.B * a.H * a.n_pages > 256) {
      const int64_t items = a.B * a.H * a.n_pages;
      DKV_KEYF_RUN(kKeyScores);
      if (with_values && VL.vec && VL.rows > 0 && items <= kSelectFuseMaxPages &&
          (items + kSelectWaves - 1) / kSelectWaves + VL.gx * VL.gy + copy_blocks_for(CP) <= 0x7fffffffLL) {
        // the selection, the value rows and the copies share one launch
        const int64_t sel_blocks = (items + kSelectWaves - 1) / kSelectWaves;
        const dim3 sgrid((unsigned)(sel_blocks + VL.gx * VL.gy + copy_blocks_for(CP)));
#define DKV_SV(B, T)                                                                                           \
  do {                                                                                                        \
    if (VL.epl == 16)                                                                                         \
      hipLaunchKernelGGL((select_pages_and_rows<B, T, 16>), sgrid, dim3(kThreads), 0, s, k, row_bytes, items,  \
                         sel_blocks, VL.p, VL.lpg, VL.row_shift, VL.gx, VL.gy, CP, copy_blocks_for(CP));    \
    else                                                                                                      \
      hipLaunchKernelGGL((select_pages_and_rows<B, T, 8>), sgrid, dim3(kThreads), 0, s, k, row_bytes, items,   \
                         sel_blocks, VL.p, VL.lpg, VL.row_shift, VL.gx, VL.gy, CP, copy_blocks_for(CP));    \
  } while (0)
#define DKV_SV_BITS(T)                    \
  do {                                    \
    if (VL.bits == 2) DKV_SV(2, T);       \
    else if (VL.bits == 4) DKV_SV(4, T);  \
    else DKV_SV(8, T);                    \
  } while (0)
        if (VL.src_dtype == kBF16) DKV_SV_BITS(kBF16);
        else if (VL.src_dtype == kF16) DKV_SV_BITS(kF16);
        else DKV_SV_BITS(kF32);
#undef DKV_SV_BITS
#undef DKV_SV
        values_done = true;
        copies_done = true;
      } else {
        hipLaunchKernelGGL(key_select_pages, dim3((unsigned)items), dim3(64), 0, s, k, row_bytes);
      }
      DKV_KEYF_RUN(kKeyCodes);
    } else {
      DKV_KEYF_RUN(kKeyAll);
    }
#undef DKV_KEYF_RUN
#undef DKV_KEYF_BITS
#undef DKV_KEYF
    return finish();
  }
  if (use_tiled) {
    const dim3 grid((unsigned)(a.B * a.H), (unsigned)a.n_pages);
    const bool select = a.key_mode == DKV_KEY_MIXED && Kp > 0 && Kp < a.D && a.selection != DKV_SELECT_GIVEN;
    if (select && row_bytes >= 4 && a.D <= kSelectMaxD) {
      // scores -> one lane per page selects -> codes
      hipLaunchKernelGGL(quantize_key_pages_tiled, grid, dim3(kThreads), tiled, s, k, kKeyScores);
      const int64_t items = a.B * a.H * a.n_pages;
      hipLaunchKernelGGL(key_select_pages, dim3((unsigned)items), dim3(64), 0, s, k, row_bytes);
      hipLaunchKernelGGL(quantize_key_pages_tiled, grid, dim3(kThreads), tiled, s, k, kKeyCodes);
    } else {
      hipLaunchKernelGGL(quantize_key_pages_tiled, grid, dim3(kThreads), tiled, s, k, kKeyAll);
    }
    return finish();
  }
  const bool f64 = a.src_dtype == kF64;
  const size_t shmem = f64 ? key_generic_smem<double>(a.D) : key_generic_smem<float>(a.D);
  DKV_CHECK(shmem <= 64 * 1024, DKV_ERR_UNSUPPORTED, "head_dim %lld is too large", (long long)a.D);
  const dim3 grid((unsigned)(a.B * a.H), (unsigned)a.n_pages);
  if (f64) {
    hipLaunchKernelGGL(quantize_key_pages_kernel<double>, grid, dim3(kThreads), shmem, s, k);
  } else {
    hipLaunchKernelGGL(quantize_key_pages_kernel<float>, grid, dim3(kThreads), shmem, s, k);
  }
  return finish();
}

extern "C" int dkv_dequantize_rows(const uint8_t* values, const void* scale, const void* zero, int meta_dtype,
                                   int64_t rows, int64_t n, int bits, int64_t group, void* out, int out_dtype,
                                   int64_t out_row_stride, void* stream) {
  DKV_CHECK(valid_meta_dtype(meta_dtype), DKV_ERR_DTYPE, "metadata dtype must be floating point");
  DKV_CHECK(valid_float_dtype(out_dtype), DKV_ERR_DTYPE, "output dtype must be f64/f32/f16/bf16");
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
  DKV_CHECK(valid_float_dtype(out_dtype), DKV_ERR_DTYPE, "output dtype must be f64/f32/f16/bf16");
  DKV_CHECK(B > 0 && H > 0 && D > 0 && tokens > 0 && group > 0, DKV_ERR_INVALID, "bad dequantize shape");
  DKV_CHECK(promoted >= 0 && promoted <= D, DKV_ERR_INVALID, "bad promoted channel count");
  DKV_CHECK(D <= 16384 && B * H <= 65535, DKV_ERR_UNSUPPORTED, "shape too large for dkv_dequantize_mixed");
  const int64_t items = tokens * D;
  hipLaunchKernelGGL(dequantize_mixed_kernel, dim3((unsigned)((items + kThreads - 1) / kThreads), (unsigned)(B * H)),
                     dim3(kThreads), (size_t)D * sizeof(int32_t), (hipStream_t)stream, low, high, idx, scale, zero,
                     meta_dtype, B, H, D, tokens, group, promoted, out, out_dtype);
  return dkv_check_launch("dkv_dequantize_mixed");
}
