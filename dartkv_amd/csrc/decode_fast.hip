// Fast single-token decode over full packed pages (gfx950, wave64).
//
// Scope: head_dim 128, 128-token pages, keys with Dart promotion (2-bit codes
// for every channel plus the upper 2 bits of NP promoted channels, one key
// group per page), 2-bit values with groups of vg (8 | vg, vg | 128) channels,
// fp16 metadata, bf16 or fp16 cache, up to 4 query heads per KV head.
// Everything else goes through the general kernel (decode.hip).
//
// One wave owns one split: a contiguous range of pages of one (batch, kv
// head).  Per page the wave
//   1. stages the packed page (10,880 bytes at the reference layout) in its
//      private LDS region with 16-byte loads; the next page is prefetched into
//      registers while the current one is processed;
//   2. builds exact-value tables: for every channel / (token, value group) the
//      dequantized value of each code under the reference's rounding chain
//      (fp16 code*scale, fp16 +zero, then the cache dtype), stored as fp16
//      (bf16 values are exact in fp16 in its normal range);
//   3. reorders channels so the NP promoted channels come first (the query is
//      permuted the same way), turning the 4-bit / 2-bit split into whole
//      16-channel blocks;
//   4. computes logits S = Q K over the page and O += P V with
//      v_mfma_f32_16x16x16f16 (query heads in the M rows, four of sixteen
//      used); the B operands are assembled in registers by v_perm lookups of
//      2-bit codes into byte-planar tables, so every K/V element is dequantized
//      exactly once;
//   5. keeps the online-softmax state (max, sum, O) across pages.
// The partial state goes to the workspace and the shared merge pass finishes.
#include <hip/hip_runtime.h>
#include <math.h>

#include "dkv_capi_util.h"
#include "dkv_decode.h"
#include "dkv_device.h"

using namespace dkv;

namespace {

typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float float4v __attribute__((ext_vector_type(4)));

constexpr int kD = 128;
constexpr int kPage = 128;
constexpr int kWaves = 4;

// Byte offsets inside one wave's LDS region (16-byte aligned; sizes depend on
// the promoted-channel count NP and value groups per token Gv).
struct LdsMap {
  int kl, vc, kh, ki, ks, kz, vs, vz, klut, klut16, vlut, pmap, qp, pt, q16, bytes;
};

__host__ __device__ inline LdsMap lds_map(int np, int gv) {
  LdsMap m;
  int o = 0;
  m.kl = o; o += 4096;            // key low codes   [128 ch][32 B]
  m.vc = o; o += 4096;            // value codes     [128 tok][32 B]
  m.kh = o; o += np * 32;         // key high codes  [NP][32 B]
  m.ki = o; o += np * 4;          // channel indices [NP] int32
  m.ks = o; o += 256;             // key scale  [128] fp16
  m.kz = o; o += 256;             // key zero   [128] fp16
  m.vs = o; o += 256 * gv;        // value scale [128 tok][Gv] fp16
  m.vz = o; o += 256 * gv;        // value zero  [128 tok][Gv] fp16
  m.klut = o; o += 1024;          // 2-bit key tables [128 pos][LO, HI]
  m.klut16 = o; o += np * 32;     // 4-bit key tables [NP][16] fp16
  m.vlut = o; o += 1024 * gv;     // value tables [Gv][128 tok][LO, HI]
  m.pmap = o; o += 128;           // position -> channel uint8
  m.qp = o; o += 1024;            // permuted query [4][128] fp16
  m.pt = o; o += 1024;            // softmax weights [4][128] fp16 (channel flags before that)
  m.q16 = o; o += 1024;           // query in channel order [4][128] fp16
  m.bytes = o;
  return m;
}


__device__ __forceinline__ uint32_t perm(uint32_t s0, uint32_t s1, uint32_t sel) {
  return __builtin_amdgcn_perm(s0, s1, sel);
}

// fp16 bit pattern of bf16(x) for an fp16 value x (round the 10-bit mantissa
// to 7 bits, nearest-even).  Exact for fp16 normal numbers; values below
// 2^-14 may differ from bf16 rounding by at most 2^-24.
__device__ __forceinline__ uint32_t round_pair_to_bf16_precision(uint32_t x) {
  const uint32_t lsb = (x >> 3) & 0x00010001u;
  return (x + 0x00030003u + lsb) & 0xfff8fff8u;
}

// Exact dequantized values for codes (c0, c1) of one (scale, zero) pair, as
// an fp16 pair: fp16(fp16(code*s) + z), then bf16 precision if requested.
__device__ __forceinline__ uint32_t lut_pair(uint32_t codes_h2, uint32_t s_h2, uint32_t z_h2, bool bf16) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  h2 c = __builtin_bit_cast(h2, codes_h2);
  h2 s = __builtin_bit_cast(h2, s_h2);
  h2 z = __builtin_bit_cast(h2, z_h2);
  h2 prod = c * s;  // -ffp-contract=off keeps the multiply and the add separate
  h2 sum = prod + z;
  uint32_t r = __builtin_bit_cast(uint32_t, sum);
  return bf16 ? round_pair_to_bf16_precision(r) : r;
}

// Byte-planar table of the 4 values for codes 0..3: LO = low bytes, HI = high bytes.
__device__ __forceinline__ void build_lut4(uint16_t s, uint16_t z, bool bf16, uint32_t* lo, uint32_t* hi) {
  const uint32_t s2 = (uint32_t)s * 0x10001u, z2 = (uint32_t)z * 0x10001u;
  const uint32_t v01 = lut_pair(0x3c000000u, s2, z2, bf16);  // codes (0, 1)
  const uint32_t v23 = lut_pair(0x42004000u, s2, z2, bf16);  // codes (2, 3)
  *lo = perm(v23, v01, 0x06040200u);
  *hi = perm(v23, v01, 0x07050301u);
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
};

struct PageAddr {
  const uint8_t *kl, *kh, *vc;
  const int32_t* ki;
  const uint16_t *ks, *kz, *vs, *vz;
};

__device__ __forceinline__ PageAddr page_addr(const dkv_segment& s, int64_t bh) {
  PageAddr p;
  p.kl = (const uint8_t*)s.key[0] + bh * s.key_bh[0];
  p.kh = (const uint8_t*)s.key[1] + bh * s.key_bh[1];
  p.ki = (const int32_t*)s.key[2] + bh * s.key_bh[2];
  p.ks = (const uint16_t*)s.key[3] + bh * s.key_bh[3];
  p.kz = (const uint16_t*)s.key[4] + bh * s.key_bh[4];
  p.vc = (const uint8_t*)s.value[0] + bh * s.value_bh[0];
  p.vs = (const uint16_t*)s.value[1] + bh * s.value_bh[1];
  p.vz = (const uint16_t*)s.value[2] + bh * s.value_bh[2];
  return p;
}

typedef __attribute__((address_space(3))) void lds_void;

// Copy `bytes` (a multiple of 16) from global `src` to LDS `dst` with
// global_load_lds_dwordx4: each instruction moves 64 x 16 bytes, lane l's
// chunk landing at dst + 16 * l.  Completion is awaited with s_waitcnt vmcnt.
__device__ __forceinline__ void copy_to_lds(uint8_t* dst, const uint8_t* src, int bytes, int lane) {
  for (int off = 0; off < bytes; off += 1024) {
    if (off + 16 * lane < bytes)
      __builtin_amdgcn_global_load_lds((const void*)(src + off + 16 * lane), (lds_void*)(dst + off), 16, 0, 0);
  }
}

// Page data in three groups, each issued as soon as the previous page no
// longer reads that LDS region.
__device__ __forceinline__ void issue_small(const LdsMap& M, uint8_t* lds, const PageAddr& a, int np, int gv,
                                            int lane) {
  copy_to_lds(lds + M.ki, (const uint8_t*)a.ki, np * 4, lane);
  copy_to_lds(lds + M.ks, (const uint8_t*)a.ks, 256, lane);
  copy_to_lds(lds + M.kz, (const uint8_t*)a.kz, 256, lane);
  copy_to_lds(lds + M.vs, (const uint8_t*)a.vs, 256 * gv, lane);
  copy_to_lds(lds + M.vz, (const uint8_t*)a.vz, 256 * gv, lane);
}
__device__ __forceinline__ void issue_keys(const LdsMap& M, uint8_t* lds, const PageAddr& a, int np, int lane) {
  copy_to_lds(lds + M.kl, a.kl, 4096, lane);
  copy_to_lds(lds + M.kh, a.kh, np * 32, lane);
}
__device__ __forceinline__ void issue_values(const LdsMap& M, uint8_t* lds, const PageAddr& a, int lane) {
  copy_to_lds(lds + M.vc, a.vc, 4096, lane);
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

// Number of copy_to_lds instructions in each staging group.
__host__ __device__ inline int n_small_loads(int np, int gv) {
  return (np * 4 + 1023) / 1024 + 2 + 2 * ((256 * gv + 1023) / 1024);
}
__host__ __device__ inline int n_key_loads(int np) { return 4 + (np * 32 + 1023) / 1024; }


// Accumulate acc[j] += a * B_j for the 8 columns j of a 4-row block whose
// B values come from 2-bit codes.
// x[m]: 16 bits = codes of the lane's 8 columns for row m (m = 0..3).
// lo[m], hi[m]: byte-planar 4-entry tables of row m.
// B_j (fp16 x4) = rows 0..3 at column j.
__device__ __forceinline__ void mma_lut_block(half4 a, const uint32_t x[4], const uint32_t lo[4], const uint32_t hi[4],
                                              float4v acc[8]) {
  const uint32_t y0 = perm(x[1], x[0], 0x05010400u);
  const uint32_t y1 = perm(x[3], x[2], 0x05010400u);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t e0 = ((y0 >> (2 * k)) & 0x03030303u) | 0x04000400u;
    const uint32_t e1 = ((y1 >> (2 * k)) & 0x03030303u) | 0x04000400u;
    const uint32_t lp0 = perm(lo[1], lo[0], e0), hp0 = perm(hi[1], hi[0], e0);
    const uint32_t lp1 = perm(lo[3], lo[2], e1), hp1 = perm(hi[3], hi[2], e1);
    const uint2 wk = make_uint2(perm(hp0, lp0, 0x05010400u), perm(hp1, lp1, 0x05010400u));
    const uint2 wk4 = make_uint2(perm(hp0, lp0, 0x07030602u), perm(hp1, lp1, 0x07030602u));
    acc[k] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, __builtin_bit_cast(half4, wk), acc[k], 0, 0, 0);
    acc[k + 4] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, __builtin_bit_cast(half4, wk4), acc[k + 4], 0, 0, 0);
  }
}

template <int GQ>
__global__ void __launch_bounds__(256, 2) decode_pages_fast(FastParams p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n = lane & 15, kq = lane >> 4;
  const int worker = blockIdx.x * kWaves + wave;
  const int total_workers = p.B * p.Hkv * p.splits;
  if (worker >= total_workers) return;
  const int split = worker % p.splits;
  const int bh = worker / p.splits;
  const int b = bh / p.Hkv, kvh = bh % p.Hkv;
  const LdsMap M = lds_map(p.np, p.gv);
  uint8_t* lds = smem + wave * M.bytes;
  const int page0 = (int)(((int64_t)split * p.count) / p.splits);
  const int page1 = (int)(((int64_t)(split + 1) * p.count) / p.splits);
  const int np = p.np, gv = p.gv;
  const bool bf16 = p.bf16 != 0;

  // running softmax state, rows r = 0..3 live in lanes 0..15
  float m_run[4], l_run[4];
  float4v O[8];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    m_run[r] = -INFINITY;
    l_run[r] = 0.f;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) O[j] = float4v{0.f, 0.f, 0.f, 0.f};

  {
    uint16_t* q16 = (uint16_t*)(lds + M.q16);
    for (int i = lane; i < GQ * kD; i += 64) {
      const int h = i / kD, c = i % kD;
      const float qv = dev_load(p.query, (int64_t)b * p.q_sb + (int64_t)(kvh * GQ + h) * p.q_sh + c, p.q_dtype);
      q16[i] = __builtin_bit_cast(uint16_t, (_Float16)qv);
    }
  }
  if (page0 < page1) {
    const PageAddr a0 = page_addr(p.segs[p.first + page0], bh);
    issue_small(M, lds, a0, np, gv, lane);
    issue_keys(M, lds, a0, np, lane);
    issue_values(M, lds, a0, lane);
  }
#pragma unroll 1
  for (int pg = page0; pg < page1; ++pg) {
    const bool has_next = pg + 1 < page1;
    PageAddr nxt;
    if (has_next) nxt = page_addr(p.segs[p.first + pg + 1], bh);
    // outstanding, oldest first: scales (this page), key codes (this page),
    // value codes (this page, 4 loads); the values may still be in flight
    vm_wait(4);

    // ---- channel order: promoted slots first, then the rest ascending ----
    uint8_t* flag = lds + M.pt;
    uint8_t* pmap = lds + M.pmap;
    const int32_t* ki = (const int32_t*)(lds + M.ki);
    flag[lane] = 0;
    flag[lane + 64] = 0;
    lds_sync();
    if (lane < np) {
      const int c = ki[lane] & 127;
      flag[c] = (uint8_t)(lane + 1);
      pmap[lane] = (uint8_t)c;
    }
    lds_sync();
    {
      const bool prom_a = flag[lane] != 0, prom_b = flag[lane + 64] != 0;
      const uint64_t rest_a = __ballot(!prom_a), rest_b = __ballot(!prom_b);
      const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
      const int ra = __popcll(rest_a & below);
      const int rb = __popcll(rest_a) + __popcll(rest_b & below);
      if (!prom_a) pmap[np + ra] = (uint8_t)lane;
      if (!prom_b) pmap[np + rb] = (uint8_t)(lane + 64);
    }
    lds_sync();

    // ---- exact-value tables ----
    const uint16_t* ks = (const uint16_t*)(lds + M.ks);
    const uint16_t* kz = (const uint16_t*)(lds + M.kz);
    uint32_t* klut = (uint32_t*)(lds + M.klut);
    for (int pos = np + lane; pos < kD; pos += 64) {
      const int c = pmap[pos];
      uint32_t lo, hi;
      build_lut4(ks[c], kz[c], bf16, &lo, &hi);
      klut[2 * pos] = lo;
      klut[2 * pos + 1] = hi;
    }
    if (lane < np) {
      const int c = pmap[lane];
      const uint32_t s2 = (uint32_t)ks[c] * 0x10001u, z2 = (uint32_t)kz[c] * 0x10001u;
      uint32_t* t16 = (uint32_t*)(lds + M.klut16 + 32 * lane);
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        // fp16 codes (2q, 2q+1)
        const _Float16 c0 = (_Float16)(2 * q), c1 = (_Float16)(2 * q + 1);
        const uint32_t codes = (uint32_t)__builtin_bit_cast(uint16_t, c0) |
                               ((uint32_t)__builtin_bit_cast(uint16_t, c1) << 16);
        t16[q] = lut_pair(codes, s2, z2, bf16);
      }
    }
    {
      const uint16_t* vs = (const uint16_t*)(lds + M.vs);
      const uint16_t* vz = (const uint16_t*)(lds + M.vz);
      uint32_t* vlut = (uint32_t*)(lds + M.vlut);
      for (int i = lane; i < kPage * gv; i += 64) {
        const int t = i / gv, g = i % gv;
        uint32_t lo, hi;
        build_lut4(vs[t * gv + g], vz[t * gv + g], bf16, &lo, &hi);
        vlut[2 * (g * kPage + t)] = lo;
        vlut[2 * (g * kPage + t) + 1] = hi;
      }
    }
    // permuted query, fp16
    {
      uint16_t* qp = (uint16_t*)(lds + M.qp);
      const uint16_t* q16 = (const uint16_t*)(lds + M.q16);
      for (int i = lane; i < GQ * kD; i += 64) {
        const int h = i / kD, pos = i % kD;
        qp[h * kD + pos] = q16[h * kD + pmap[pos]];
      }
    }
    lds_sync();
    if (has_next) issue_small(M, lds, nxt, np, gv, lane);

    // ---- S = Q K over the page (columns: token 8n + j) ----
    float4v S[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) S[j] = float4v{0.f, 0.f, 0.f, 0.f};
    const uint8_t* kl = lds + M.kl;
    const uint8_t* kh = lds + M.kh;
    const uint16_t* klut16 = (const uint16_t*)(lds + M.klut16);
#pragma unroll 1
    for (int blk = 0; blk < kD / 16; ++blk) {
      const int pos0 = blk * 16 + 4 * kq;
      half4 a = half4{0, 0, 0, 0};
      if (n < GQ) a = *(const half4*)(lds + M.qp + 2 * (n * kD + pos0));
      if (blk * 16 < np) {
        // promoted channels: 4-bit codes, one table lookup per element
        uint32_t xl[4], xh[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const int c = pmap[pos0 + m];
          xl[m] = *(const uint16_t*)(kl + 32 * c + 2 * n);
          xh[m] = *(const uint16_t*)(kh + 32 * (pos0 + m) + 2 * n);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          uint16_t v[4];
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            const uint32_t code = ((xl[m] >> (2 * j)) & 3u) | (((xh[m] >> (2 * j)) & 3u) << 2);
            v[m] = klut16[(pos0 + m) * 16 + code];
          }
          uint2 w = make_uint2((uint32_t)v[0] | ((uint32_t)v[1] << 16), (uint32_t)v[2] | ((uint32_t)v[3] << 16));
          S[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, __builtin_bit_cast(half4, w), S[j], 0, 0, 0);
        }
      } else {
        uint32_t x[4], lo[4], hi[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const int c = pmap[pos0 + m];
          x[m] = *(const uint16_t*)(kl + 32 * c + 2 * n);
          const uint2 t = *(const uint2*)(klut + 2 * (pos0 + m));
          lo[m] = t.x;
          hi[m] = t.y;
        }
        mma_lut_block(a, x, lo, hi, S);
      }
    }
    lds_sync();
    if (has_next) issue_keys(M, lds, nxt, np, lane);

    // ---- online softmax (rows r < GQ in lanes 0..15) ----
    float alpha[4];
    {
      uint16_t* pt = (uint16_t*)(lds + M.pt);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float mx = -INFINITY;
#pragma unroll
        for (int j = 0; j < 8; ++j) mx = fmaxf(mx, S[j][r] * p.scale);
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
        const float m_new = fmaxf(m_run[r], mx);
        alpha[r] = __expf(m_run[r] - m_new);
        float sum = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float w = __expf(S[j][r] * p.scale - m_new);
          sum += w;
          if (kq == 0 && r < GQ) pt[r * kPage + 8 * n + j] = __builtin_bit_cast(uint16_t, (_Float16)w);
        }
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) sum += __shfl_xor(sum, off, 64);
        l_run[r] = l_run[r] * alpha[r] + sum;
        m_run[r] = m_new;
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
#pragma unroll
      for (int r = 0; r < 4; ++r) O[j][r] *= alpha[r];
    }
    lds_sync();

    // this page's value codes are older than the next page's scale and key
    // loads issued since
    vm_wait(has_next ? n_small_loads(np, gv) + n_key_loads(np) : 0);

    // ---- O += P V (columns: channel 8n + j) ----
    const uint8_t* vc = lds + M.vc;
    const uint32_t* vlut = (const uint32_t*)(lds + M.vlut);
    const int g = (8 * n) / p.vg;
#pragma unroll 1
    for (int blk = 0; blk < kPage / 16; ++blk) {
      const int t0 = blk * 16 + 4 * kq;
      half4 a = half4{0, 0, 0, 0};
      if (n < GQ) a = *(const half4*)(lds + M.pt + 2 * (n * kPage + t0));
      uint32_t x[4], lo[4], hi[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        x[m] = *(const uint16_t*)(vc + 32 * (t0 + m) + 2 * n);
        const uint2 t = *(const uint2*)(vlut + 2 * (g * kPage + t0 + m));
        lo[m] = t.x;
        hi[m] = t.y;
      }
      mma_lut_block(a, x, lo, hi, O);
    }
    lds_sync();
    if (has_next) issue_values(M, lds, nxt, lane);
  }

  // ---- partial state ----
  if (lane < 16) {
#pragma unroll
    for (int r = 0; r < GQ; ++r) {
      const int hq = kvh * GQ + r;
      float* rec = p.ws + (((int64_t)b * p.Hq + hq) * p.split_stride + split) * (kD + 2);
      if (lane == 0) {
        rec[0] = m_run[r];
        rec[1] = l_run[r];
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) rec[2 + 8 * n + j] = O[j][r];
    }
  }
}

}  // namespace

namespace dkv {

int fast_decode_max_loads(int np, int gv) { return n_small_loads(np, gv) + n_key_loads(np); }

size_t fast_decode_lds_bytes(int np, int gv) { return (size_t)kWaves * lds_map(np, gv).bytes; }

int launch_fast_decode(const dkv_decode_args& a, int first, int count, int np, int vg, int splits, int split_stride,
                       hipStream_t stream) {
  FastParams p;
  p.segs = a.segments;
  p.first = first;
  p.count = count;
  p.B = (int)a.B;
  p.Hq = (int)a.Hq;
  p.Hkv = (int)a.Hkv;
  p.GQ = (int)(a.Hq / a.Hkv);
  p.splits = splits;
  p.split_stride = split_stride;
  p.np = np;
  p.vg = vg;
  p.gv = kD / vg;
  p.bf16 = a.cache_dtype == kBF16 ? 1 : 0;
  p.scale = (float)a.scale;
  p.query = a.query;
  p.q_dtype = (int)a.q_dtype;
  p.q_sb = a.q_sb;
  p.q_sh = a.q_sh;
  p.ws = (float*)a.workspace;
  const int64_t workers = (int64_t)p.B * p.Hkv * splits;
  const unsigned blocks = (unsigned)((workers + kWaves - 1) / kWaves);
  const size_t lds = fast_decode_lds_bytes(np, p.gv);
  switch (p.GQ) {
    case 1:
      hipLaunchKernelGGL(decode_pages_fast<1>, dim3(blocks), dim3(256), lds, stream, p);
      break;
    case 2:
      hipLaunchKernelGGL(decode_pages_fast<2>, dim3(blocks), dim3(256), lds, stream, p);
      break;
    case 4:
      hipLaunchKernelGGL(decode_pages_fast<4>, dim3(blocks), dim3(256), lds, stream, p);
      break;
    default:
      set_error("fast decode supports 1, 2 or 4 query heads per KV head");
      return DKV_ERR_UNSUPPORTED;
  }
  return dkv_check_launch("dkv_decode_attention(fast pages)");
}

}  // namespace dkv
