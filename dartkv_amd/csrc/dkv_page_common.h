// Helpers shared by the MFMA page kernels (gfx950, wave64): LDS staging with
// LDS DMA, counted waits, page descriptors, byte permutes and wave reductions.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dkv_capi_util.h"
#include "dkv_decode.h"
#include "dkv_dense.h"
#include "dkv_device.h"

namespace {

using namespace dkv;

typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));

constexpr int kD = 128;
constexpr int kPage = 128;
constexpr int kWaves = 4;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kSlack = 8.f;  // log2 headroom before the running max moves
__device__ __forceinline__ uint32_t perm(uint32_t s0, uint32_t s1, uint32_t sel) {
  return __builtin_amdgcn_perm(s0, s1, sel);
}

// Constants in registers the compiler cannot see through.  gfx9 VOP3
// encodings take no literal and one scalar operand, so with two literal
// constants (x & m) | c becomes v_and + v_or; with m in a scalar register and c
// in a vector register it is one v_and_or_b32.  Made once per kernel.
__device__ __forceinline__ uint32_t in_sgpr(uint32_t v) {
  uint32_t r;
  asm("s_mov_b32 %0, %1" : "=s"(r) : "i"(v));
  return r;
}
__device__ __forceinline__ uint32_t in_vgpr(uint32_t v) {
  uint32_t r;
  asm("v_mov_b32 %0, %1" : "=v"(r) : "i"(v));
  return r;
}

// fp16 bit pattern of bf16(x) for an fp16 value x (round the 10-bit mantissa
// to 7 bits, nearest-even).  Exact for fp16 normal numbers; values below
// 2^-14 may differ from bf16 rounding by at most 2^-24.
__device__ __forceinline__ uint32_t round_pair_to_bf16_precision(uint32_t x) {
  const uint32_t lsb = (x >> 3) & 0x00010001u;
  return (x + 0x00030003u + lsb) & 0xfff8fff8u;
}

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// fp16 scale or zero point (bits in the low half of x) in both halves; as an
// operand of a packed op this is an op_sel broadcast, not an instruction.
__device__ __forceinline__ half2v splat_h(uint32_t x) {
  const _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)x);
  return half2v{h, h};
}

// Exact dequantized values for codes (c0, c1) of one (scale, zero) pair, as
// an fp16 pair: fp16(fp16(code*s) + z), then bf16 precision if BF16.
template <bool BF16>
__device__ __forceinline__ uint32_t lut_pair(uint32_t codes_h2, half2v s, half2v z) {
  const half2v c = __builtin_bit_cast(half2v, codes_h2);
  const half2v prod = c * s;  // -ffp-contract=off keeps the multiply and the add separate
  const half2v sum = prod + z;
  uint32_t r = __builtin_bit_cast(uint32_t, sum);
  return BF16 ? round_pair_to_bf16_precision(r) : r;
}

// Codes (2q + 8h, 2q + 1 + 8h) as an fp16 pair (h = 0, 1: entries 0..7 or 8..15).
__device__ __forceinline__ uint32_t code_pair(int q, int h) {
  const uint32_t lo[4] = {0x3c000000u, 0x42004000u, 0x45004400u, 0x47004600u};  // (0, 1) .. (6, 7)
  const uint32_t hi[4] = {0x48804800u, 0x49804900u, 0x4a804a00u, 0x4b804b00u};  // (8, 9) .. (14, 15)
  return h ? hi[q] : lo[q];
}

// Four entries (fp16) of LDS tables, at byte offsets off + byte j of sel from
// base (whose low byte is zero, so a byte permute forms each address), as a
// B operand.
__device__ __forceinline__ half4 gather4(uint32_t base, uint32_t sel, int off) {
  typedef __attribute__((address_space(3))) const _Float16 lds_half;
  half4 r;
#pragma unroll
  for (int j = 0; j < 4; ++j) r[j] = ((lds_half*)(uintptr_t)perm(base, sel, 0x07060500u | j))[off / 2];
  return r;
}

struct FastParams {
  const dkv_segment* segs;   // descriptor table; pages are entries [first, first + count)
  int first, count;
  int B, Hq, Hkv, GQ;
  int splits;                // splits per (batch, kv head) for this kernel
  int split_stride;          // total splits in the workspace record
  int np;                    // promoted channels (multiple of 16)
  int vg, gv;                // value group size / groups per token
  int bf16;                  // cache dtype is bf16
  float scale;
  const void* query;
  int q_dtype;
  int64_t q_sb, q_sh;
  float* ws;
  // With a dense rest in the launch (dense_workers > 0), the workers past the
  // page workers run its chunks (dense_worker) and write their records.
  int dense_chunks, dense_workers;
  DecodeParams rest;
};

// Host side: the dense-rest fields of a page kernel's parameters (none when
// f is null).  Call after p.B and p.Hkv are set.
inline void set_fused(FastParams& p, const FusedRest* f) {
  p.dense_chunks = p.dense_workers = 0;
  if (f == nullptr) return;
  p.rest = *f->rest;
  p.dense_chunks = f->chunks;
  p.dense_workers = p.B * p.Hkv * p.rest.n_total * f->chunks;
}

// Dense-rest worker dw of a page kernel launch: chunk dw % (n_total * chunks)
// of (batch, kv head) dw / (n_total * chunks), with the wave's LDS region.
template <int MG, bool BF>
__device__ __forceinline__ void dense_worker(const FastParams& p, int dw, int lane, float* lds) {
  if (dw >= p.dense_workers) return;
  const int per_bh = p.rest.n_total * p.dense_chunks;
  const int bhi = dw / per_bh, t = dw % per_bh;
  dense_chunk<MG, BF>(p.rest, p.dense_chunks, bhi, t / p.dense_chunks, t % p.dense_chunks, lane, lds,
                      lds + kDenseDim * MG);
}

// A gathered copy's lanes move from one page field to another (possibly in
// another allocation) by wave-uniform byte distances; the addresses are
// formed as integers, which pointer arithmetic across objects does not express.
__device__ __forceinline__ int64_t byte_gap(const void* to, const void* from) {
  return (int64_t)((uintptr_t)to - (uintptr_t)from);
}
__device__ __forceinline__ const uint8_t* byte_at(const void* base, int64_t off) {
  return (const uint8_t*)((uintptr_t)base + (uint64_t)off);
}

struct PageAddr {
  const uint8_t *kl, *kh, *vc;
  const int32_t* ki;
  const uint16_t *ks, *kz, *vs, *vz;
};

// The descriptor is the same for the whole wave: it is read through the
// constant address space (scalar loads) and its fields are kept in scalar
// registers, so the address arithmetic runs on the scalar unit.
typedef __attribute__((address_space(4))) const dkv_segment const_segment;

__device__ __forceinline__ const_segment& descriptor(const dkv_segment* table, int i) {
  return ((const_segment*)table)[i];
}

__device__ __forceinline__ uint64_t uniform_u64(uint64_t x) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(x >> 32));
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ PageAddr page_addr(const_segment& s, int64_t bh) {
  PageAddr p;
  p.kl = (const uint8_t*)uniform_u64(s.key[0] + (uint64_t)(bh * (int64_t)uniform_u64((uint64_t)s.key_bh[0])));
  p.kh = (const uint8_t*)uniform_u64(s.key[1] + (uint64_t)(bh * (int64_t)uniform_u64((uint64_t)s.key_bh[1])));
  p.ki = (const int32_t*)uniform_u64(s.key[2] + (uint64_t)(4 * bh * (int64_t)uniform_u64((uint64_t)s.key_bh[2])));
  p.ks = (const uint16_t*)uniform_u64(s.key[3] + (uint64_t)(2 * bh * (int64_t)uniform_u64((uint64_t)s.key_bh[3])));
  p.kz = (const uint16_t*)uniform_u64(s.key[4] + (uint64_t)(2 * bh * (int64_t)uniform_u64((uint64_t)s.key_bh[4])));
  p.vc = (const uint8_t*)uniform_u64(s.value[0] + (uint64_t)(bh * (int64_t)uniform_u64((uint64_t)s.value_bh[0])));
  p.vs = (const uint16_t*)uniform_u64(s.value[1] + (uint64_t)(2 * bh * (int64_t)uniform_u64((uint64_t)s.value_bh[1])));
  p.vz = (const uint16_t*)uniform_u64(s.value[2] + (uint64_t)(2 * bh * (int64_t)uniform_u64((uint64_t)s.value_bh[2])));
  return p;
}

// Two K = 16 blocks in one v_mfma_f32_16x16x32_f16: lane (n, kq) holds K
// indices 8 kq .. 8 kq + 7, so concatenating each lane's operands of blocks
// u and v gives K index 8 kq + i = block u's 4 kq + i for i < 4 and block v's
// 4 kq + i - 4 otherwise; the product is the sum of the two blocks' products.
__device__ __forceinline__ half8 cat8(half4 u, half4 v) {
  return __builtin_shufflevector(u, v, 0, 1, 2, 3, 4, 5, 6, 7);
}
__device__ __forceinline__ float4v mma2(half4 a0, half4 a1, half4 b0, half4 b1, float4v acc) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(cat8(a0, a1), cat8(b0, b1), acc, 0, 0, 0);
}

typedef __attribute__((address_space(3))) void lds_void;

// Copy `bytes` (a multiple of 16) from global `src` to LDS `dst` with
// global_load_lds_dwordx4: each instruction moves 64 x 16 bytes, lane l's
// chunk landing at dst + 16 * l.  Completion is awaited with vm_wait(n),
// which counts these instructions.  They are issued from inline assembly so
// the compiler does not track them: its conservative aliasing of LDS DMA
// against every later LDS store would otherwise insert vmcnt(0) before the
// table writes of the next page and stall on the prefetch this overlaps.
// (M0 holds the LDS destination; one wait state between writing M0 and the
// load.)
__device__ __forceinline__ void dma16(const uint8_t* src, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds_addr) : "memory");
}
__device__ __forceinline__ void copy_to_lds(uint8_t* dst, const uint8_t* src, int bytes, int lane) {
  const uint32_t base = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void*)dst);
  for (int off = 0; off < bytes; off += 1024) {
    if (off + 16 * lane < bytes) dma16(src + off + 16 * lane, base + off);
  }
}

// All LDS traffic of this wave done (cross-lane LDS hand-off within the wave).
__device__ __forceinline__ void lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
// Wait until at most n vector-memory operations of this wave are outstanding
// (loads complete in issue order), and until all LDS traffic is done.
// gfx9 s_waitcnt encoding: vmcnt[3:0] in bits 3:0, expcnt in 6:4 (7 = no
// wait), lgkmcnt in 11:8 (0 = wait for all).  n must be < 16.
__device__ __forceinline__ void vm_wait(int n) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  switch (n) {
    case 0: __builtin_amdgcn_s_waitcnt(0x0070); break;
    case 1: __builtin_amdgcn_s_waitcnt(0x0071); break;
    case 2: __builtin_amdgcn_s_waitcnt(0x0072); break;
    case 3: __builtin_amdgcn_s_waitcnt(0x0073); break;
    case 4: __builtin_amdgcn_s_waitcnt(0x0074); break;
    case 5: __builtin_amdgcn_s_waitcnt(0x0075); break;
    case 6: __builtin_amdgcn_s_waitcnt(0x0076); break;
    case 7: __builtin_amdgcn_s_waitcnt(0x0077); break;
    case 8: __builtin_amdgcn_s_waitcnt(0x0078); break;
    case 9: __builtin_amdgcn_s_waitcnt(0x0079); break;
    case 10: __builtin_amdgcn_s_waitcnt(0x007a); break;
    case 11: __builtin_amdgcn_s_waitcnt(0x007b); break;
    case 12: __builtin_amdgcn_s_waitcnt(0x007c); break;
    case 13: __builtin_amdgcn_s_waitcnt(0x007d); break;
    case 14: __builtin_amdgcn_s_waitcnt(0x007e); break;
    case 15: __builtin_amdgcn_s_waitcnt(0x007f); break;
    default: __builtin_amdgcn_s_waitcnt(0x0070); break;
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ _Float16 lds_h(const uint8_t* base, int off) { return *(const _Float16*)(base + off); }
__device__ __forceinline__ uint32_t lds_u32(const uint8_t* base, int off) { return *(const uint32_t*)(base + off); }

// A operand: half i read from byte offset a[i] + off; a[i] points into the
// query / weight rows for the lane's own slot and into the zero block otherwise.
__device__ __forceinline__ half4 load_a(const uint8_t* lds, const int a[4], int off) {
  half4 r;
  r[0] = lds_h(lds, a[0] + off);
  r[1] = lds_h(lds, a[1] + off);
  r[2] = lds_h(lds, a[2] + off);
  r[3] = lds_h(lds, a[3] + off);
  return r;
}

// Slot-layout A operand from its one non-zero value: v (16 bits) at half
// `slot` of the four, zeros elsewhere, by two byte permutes with lane-constant
// selectors (slot_sel; all zero bytes for a lane without a row).
__device__ __forceinline__ half4 slot_a(uint32_t v, uint2 sel) {
  return __builtin_bit_cast(half4, make_uint2(perm(0u, v, sel.x), perm(0u, v, sel.y)));
}
__device__ __forceinline__ uint2 slot_sel(int slot, bool row) {
  const uint32_t z = 0x0c0c0c0cu, at_lo = 0x0c0c0100u, at_hi = 0x01000c0cu;  // 0x0c: a zero byte
  if (!row) return make_uint2(z, z);
  return make_uint2(slot == 0 ? at_lo : slot == 1 ? at_hi : z, slot == 2 ? at_lo : slot == 3 ? at_hi : z);
}

__device__ __forceinline__ float wave_max64(float v) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}
__device__ __forceinline__ float wave_sum64(float v) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ __forceinline__ float uniform(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v)));
}

// Power-of-two exponent e that brings the largest |q| of the wave's query
// elements (N per lane) into [2^14, 2^15): fp16 then holds q * 2^-e at full
// precision, and the logit scale takes 2^e back exactly.  Zero for an all-zero
// query or one whose largest element is infinite (NaN elements are ignored
// here and propagate through the products).
template <int N>
__device__ __forceinline__ int query_exponent(const float (&qv)[N]) {
  float amax = 0.f;
#pragma unroll
  for (int r = 0; r < N; ++r) amax = fmaxf(amax, fabsf(qv[r]));
  amax = uniform(wave_max64(amax));
  if (!(amax > 0.f) || amax == INFINITY) return 0;
  return __builtin_amdgcn_readfirstlane(ilogbf(amax) - 14);
}


}  // namespace
