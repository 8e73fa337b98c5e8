// Fast single-token decode over full packed pages (gfx950, wave64).
//
// Scope: head_dim 128, 128-token pages, keys with Dart promotion (2-bit codes
// for every channel plus the upper 2 bits of NP promoted channels, one key
// group per page), 2-bit values with groups of vg (16 | vg, vg | 128)
// channels, fp16 metadata, bf16 or fp16 cache, 1, 2, 4, 8 or 16 query rows per
// KV head (8 or 16 rows: two or four row groups of 4, each with its own Q K
// MFMAs on the same dequantized B operands; the multi-token path maps two or
// four tokens of a 4-head group here).  Everything else goes through the general kernel
// (decode.hip).
//
// One wave owns one split: a contiguous range of pages of one (batch, kv
// head).  (Launches that leave most of the GPU idle give a split four waves,
// each a quarter of the page's channels: "channel-split pages" below.)  Per
// page the wave
//   1. stages the packed page (10,880 bytes at the reference layout) in its
//      private LDS region with global_load_lds; the next page's parts are
//      issued as soon as the current page no longer reads their region;
//   2. builds exact-value tables: for every channel / (token, value group) the
//      dequantized value of each code under the reference's rounding chain
//      (fp16 code*scale, fp16 +zero, then the cache dtype), stored as fp16
//      (bf16 values are exact in fp16 in its normal range) in byte planes
//      (low bytes of the entries in one dword, high bytes in another), and a
//      16-entry table per promoted channel;
//   3. computes S = Q K with f16 MFMAs (16x16, K = 32: two 16-deep blocks per
//      instruction) in a "slot" layout: the 16 rows of a tile are 4 slots x 4
//      query heads, the 16 K values of one MFMA are 4 channels x 4 slots and a
//      slot picks one of 4 tokens, so the B values a lane holds are 4 tokens of
//      ONE channel (one table, four v_perm lookups of the 2-bit codes) and the
//      A operand carries q at the lane's slot and zeros elsewhere.  The
//      promoted channels' 2-bit tables are zero; a second pass adds their
//      4-bit products, each B element one 2-byte LDS gather from the channel's
//      16-entry table at an address formed by byte permutes;
//   4. keeps an online softmax in base 2 whose running max only moves when a
//      logit exceeds it by more than 8 (so p <= 256 keeps fp16's relative
//      precision); row sums stay per lane until the end;
//   5. computes O += P V with the query heads in the MFMA rows and 16 tokens
//      per K block, the weights written to LDS in the blocks' K order and the
//      value B operands looked up in the (token, group) tables.
// The partial state goes to the workspace and the shared merge pass finishes.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdlib.h>

#include <atomic>

#include "dkv_capi_util.h"
#include "dkv_decode.h"
#include "dkv_device.h"
#include "dkv_page_common.h"

using namespace dkv;

namespace {

constexpr int kQpStride = 264;     // bytes between promoted-query rows (8 banks + 2 apart)
constexpr int kPtStride = 288;     // bytes between softmax-weight rows (8 banks apart)
constexpr int kVlutStride = 1056;  // bytes between value-table groups (8 banks apart)

// Byte offsets inside one wave's LDS region (16-byte aligned; sizes depend on
// the promoted-channel count NP and value groups per token Gv).
struct LdsMap {
  int kl, vc, kh, ki, ks, kz, vs, vz, klut, klut16, vlut, pidx, q16, qp, pt, zero, bytes;
};

// rg: row groups of 4 query rows (1, or 2 / 4 for 8 / 16 rows per KV head).
// With several, the promoted channels' query rows live in the softmax-weight
// region (which is free from the weights' last read in P V until the softmax
// writes them) and the query takes 4 rg rows.
__host__ __device__ inline LdsMap lds_map(int np, int gv, int rg) {
  LdsMap m;
  int o = 0;
  // Fields whose offsets depend only on NP come first, so they are
  // compile-time constants in the kernel; the Gv-dependent ones follow.
  m.kl = o; o += 4096;                     // key low codes   [128 ch][32 B]
  m.vc = o; o += 4096;                     // value codes     [128 tok][32 B]
  m.kh = o; o += np * 32;                  // key high codes  [NP][32 B]
  m.ki = o; o += (np * 4 + 15) / 16 * 16;  // channel indices [NP] int32
  m.ks = o; o += 256;                      // key scale  [128] fp16
  m.kz = o; o += 256;                      // key zero   [128] fp16
  m.klut = o; o += 1024;                   // 2-bit key tables [128 ch][LO, HI] (zero for promoted channels), key_slot order
  o = (o + 255) / 256 * 256;               // (the 4-bit tables are addressed by byte: 256-aligned)
  m.klut16 = o; o += np * 32;              // 4-bit key tables [NP][16] fp16
  m.pidx = o; o += 64;                     // promoted channels [NP] uint8 (a copy: ki is refilled early)
  m.q16 = o; o += 1024 * rg;               // query [4 rg][128 ch] fp16
  // A-operand sources; row strides put the rows one read touches in distinct
  // banks, and the zero block 16 banks after an aligned row start.
  o = (o + 127) / 128 * 128;
  if (rg == 1) {
    m.qp = o; o += 4 * kQpStride;          // query of the promoted channels [4][NP] fp16
    o = (o + 127) / 128 * 128;
  }
  m.pt = o; o += 4 * rg * kPtStride;       // softmax weights [4 rg][128 tok] fp16
  if (rg != 1) m.qp = m.pt;                // [4 rg][NP] fits: kQpStride <= kPtStride
  o = (o + 127) / 128 * 128 + 64;
  m.zero = o; o += 256;                    // zeros read by A-operand lanes without data
  o = (o + 15) / 16 * 16;
  m.vs = o; o += 256 * gv;                 // value scale [128 tok][Gv] fp16
  m.vz = o; o += 256 * gv;                 // value zero  [128 tok][Gv] fp16
  m.vlut = o; o += kVlutStride * gv;       // value tables [Gv][128 tok][LO, HI] in K order (kpos), padded rows
  m.bytes = (o + 255) / 256 * 256;         // keeps every wave's region 256-aligned
  return m;
}

// Position of channel c's 2-bit key table: the tables of channels 8u + kq and
// 8u + 4 + kq (channel blocks 2u and 2u + 1 of lane group kq) are adjacent, so
// one 16-byte read serves a pair of blocks.
__host__ __device__ inline int key_slot(int c) { return (c & ~7) | ((c & 3) << 1) | ((c >> 2) & 1); }

// K position of token t in a P V block (block t / 16, K index 4 (t % 4) + (t / 4) % 4):
// the softmax weights and the value tables are stored in this order, so a
// lane's four tokens t, t + 4, t + 8, t + 12 are adjacent.
__host__ __device__ inline int kpos(int t) { return (t & ~15) | ((t & 3) << 2) | ((t >> 2) & 3); }

// Byte-plane table of the 4 values for codes 0..3: x = low bytes, y = high bytes.
// For codes 0 and 1 the products 0 * s and 1 * s are exact, so one fused
// multiply-add rounds once, exactly as fp16(fp16(code * s) + z) does; codes 2
// and 3 multiply and add separately.
template <bool BF16>
__device__ __forceinline__ uint2 build_lut4(uint32_t s, uint32_t z) {
  const half2v sv = splat_h(s), zv = splat_h(z);
  uint32_t v01 = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(half2v{0.0f16, 1.0f16}, sv, zv));
  if (BF16) v01 = round_pair_to_bf16_precision(v01);
  const uint32_t v23 = lut_pair<BF16>(0x42004000u, sv, zv);  // codes (2, 3)
  return make_uint2(perm(v23, v01, 0x06040200u), perm(v23, v01, 0x07050301u));
}

// B operand (4 fp16 = slots 0..3 of one table) from 4 codes e (one per byte,
// values 0..3) and a byte-plane table (lo, hi).
__device__ __forceinline__ half4 lookup4(uint32_t e, uint32_t lo, uint32_t hi) {
  const uint32_t l4 = perm(hi, lo, e);  // selector bytes 0..3 pick from lo
  const uint32_t h4 = perm(lo, hi, e);  // ... and here from hi
  return __builtin_bit_cast(half4, make_uint2(perm(h4, l4, 0x05010400u), perm(h4, l4, 0x07030602u)));
}

// B operand from 4-bit codes by LDS gathers: wl / wh = the low / high code
// dwords (bits 8j + sh, 8j + sh + 1 of byte j hold the lane's token of byte
// j); rl = (sh - 1) & 31 and rh = (sh - 3) & 31 rotate them to 2 x low and
// 8 x high, so byte j of sel = 2 code_j + 32 kq (kq32 = 32 kq in every byte)
// is the byte offset of the entry in the lane's table (slot 4 pb + kq).  tab
// is the LDS address of the block's tables with its low byte zero, so a byte
// permute forms each element's address.  m6 = 0x06060606 and m18 = 0x18181818
// in scalar registers.
__device__ __forceinline__ half4 gather16(uint32_t wl, uint32_t wh, uint32_t rl, uint32_t rh, uint32_t kq32,
                                          uint32_t tab, int off, uint32_t m6, uint32_t m18) {
  typedef __attribute__((address_space(3))) const _Float16 lds_half;
  const uint32_t x = (__builtin_amdgcn_alignbit(wl, wl, rl) & m6) | kq32;
  const uint32_t sel = (__builtin_amdgcn_alignbit(wh, wh, rh) & m18) | x;
  half4 r;
#pragma unroll
  for (int j = 0; j < 4; ++j) r[j] = ((lds_half*)(uintptr_t)perm(tab, sel, 0x07060500u | j))[off / 2];
  return r;
}

// Page data in three groups, each issued as soon as the previous page no
// longer reads that LDS region.
//
// The small fields take as few copies as their bytes allow: each lane of a
// copy reads its own 16 bytes and lands them at M0 + 16 lane, so one copy
// gathers several fields into adjacent LDS regions (promoted-channel indices,
// key scales and key zero points in one; value scales and zero points in
// 512 gv / 1024 more).  A wave pays for every copy it issues, partial or not,
// whatever their bytes, so five partial copies cost more than two.
__device__ __forceinline__ void issue_small(const LdsMap& M, uint8_t* lds, const PageAddr& a, int np, int gv,
                                            int lane) {
  const int ni = (np * 4 + 15) / 16;  // 16-byte lanes of the indices: M.ks = M.ki + 16 ni, M.kz = M.ks + 256
  {
    // lane -> its field's base plus 16 (lane - first lane of the field), as
    // wave-uniform byte distances (a select chain became a table in scratch)
    const uint32_t dst = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void*)(lds + M.ki));
    const int64_t to_ks = byte_gap(a.ks, a.ki) - 16 * ni;
    const int64_t to_kz = byte_gap(a.kz, a.ks) - 256;
    const uint8_t* src = byte_at(a.ki, 16 * lane + (lane >= ni ? to_ks : 0) + (lane >= ni + 16 ? to_kz : 0));
    if (lane < ni + 32) dma16(src, dst);
  }
  const uint32_t dst = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void*)(lds + M.vs));  // M.vz = M.vs + 256 gv
  for (int off = 0; off < 512 * gv; off += 1024) {
    const int i = (off >> 4) + lane;
    const int64_t to_vz = byte_gap(a.vz, a.vs) - 256 * gv;
    if (i < 32 * gv) dma16(byte_at(a.vs, 16 * i + (i >= 16 * gv ? to_vz : 0)), dst + off);
  }
}
__device__ __forceinline__ void issue_keys(const LdsMap& M, uint8_t* lds, const PageAddr& a, int np, int lane) {
  copy_to_lds(lds + M.kl, a.kl, 4096, lane);
  copy_to_lds(lds + M.kh, a.kh, np * 32, lane);
}
__device__ __forceinline__ void issue_values(const LdsMap& M, uint8_t* lds, const PageAddr& a, int lane) {
  copy_to_lds(lds + M.vc, a.vc, 4096, lane);
}

// Number of copy_to_lds instructions in each staging group.
__host__ __device__ inline int n_small_loads(int np, int gv) { return 1 + (512 * gv + 1023) / 1024; }
__host__ __device__ inline int n_key_loads(int np) { return 4 + (np * 32 + 1023) / 1024; }

// 4-bit key tables of the NP promoted slots: lanes (2j, 2j+1) build entries
// 0..7 / 8..15 of slot j (16 fp16 entries per slot).
template <bool BF16, int NP>
__device__ __forceinline__ void build_lut16_tables(const LdsMap& M, uint8_t* lds, const uint16_t* ks,
                                                   const uint16_t* kz, int lane) {
  const uint8_t* pidx = lds + M.pidx;
#pragma unroll
  for (int j0 = 0; j0 < NP; j0 += 32) {
    const int j = j0 + (lane >> 1);
    if (j < NP) {
      const int half = lane & 1;
      const int c = pidx[j];
      const half2v s2 = splat_h(ks[c]), z2 = splat_h(kz[c]);
      // fp16 code pairs (8 half + 2q, 8 half + 2q + 1), q = 0..3
      const uint32_t e0 = half ? 0x48804800u : 0x3c000000u;  // (8, 9)   | (0, 1)
      const uint32_t e1 = half ? 0x49804900u : 0x42004000u;  // (10, 11) | (2, 3)
      const uint32_t e2 = half ? 0x4a804a00u : 0x45004400u;  // (12, 13) | (4, 5)
      const uint32_t e3 = half ? 0x4b804b00u : 0x47004600u;  // (14, 15) | (6, 7)
      const uint32_t v0 = lut_pair<BF16>(e0, s2, z2), v1 = lut_pair<BF16>(e1, s2, z2);
      const uint32_t v2 = lut_pair<BF16>(e2, s2, z2), v3 = lut_pair<BF16>(e3, s2, z2);
      *(uint4*)(lds + M.klut16 + 32 * j + 16 * half) = make_uint4(v0, v1, v2, v3);
    }
  }
}

// O[j] += a * B_j for the 8 channel tiles j of one 16-token block in the
// heads-in-rows layout (rows 0..3 = query heads, K = 4 tokens per lane).
// x[m]: 16 bits = codes of the lane's 8 channels for token row m (m = 0..3);
// lo[m], hi[m]: byte-plane tables of token row m.  Rows m and m + 1 share one
// v_perm: selector bit 2 picks the second row's table.  m3 = 0x03030303 in a
// scalar register, sel2 = 0x04000400 in a vector register.  All eight B
// operands are formed before the MFMAs issue, so no MFMA waits on the VALU
// result it reads.
// wk[j]: the B operand of channel tile j (j < 8).  With W = 4 (a channel-split
// wave) only tiles k0 and k0 + 4, as wk[0] and wk[1].
template <int W>
__device__ __forceinline__ void lut_block_operands(const uint32_t x[4], const uint32_t lo[4], const uint32_t hi[4],
                                                   uint2 wk[8 / W], uint32_t m3, uint32_t sel2, int k0) {
  const uint32_t y0 = perm(x[1], x[0], 0x05010400u);
  const uint32_t y1 = perm(x[3], x[2], 0x05010400u);
#pragma unroll
  for (int kk = 0; kk < 4 / W; ++kk) {
    const int k = W > 1 ? k0 : kk;
    const uint32_t e0 = ((y0 >> (2 * k)) & m3) | sel2;
    const uint32_t e1 = ((y1 >> (2 * k)) & m3) | sel2;
    const uint32_t lp0 = perm(lo[1], lo[0], e0), hp0 = perm(hi[1], hi[0], e0);
    const uint32_t lp1 = perm(lo[3], lo[2], e1), hp1 = perm(hi[3], hi[2], e1);
    wk[kk] = make_uint2(perm(hp0, lp0, 0x05010400u), perm(hp1, lp1, 0x05010400u));
    wk[kk + 4 / W] = make_uint2(perm(hp0, lp0, 0x07030602u), perm(hp1, lp1, 0x07030602u));
  }
}


// Channel-split pages (W = 4, for launches that leave most of the GPU idle):
// the four waves of a workgroup take one split together.  Each stages the
// whole page and builds every table, but takes a quarter of the work that
// scales with channels: Q K channel blocks 8 w .. 8 w + 7, the promoted pairs
// w, w + 4, ... and the P V outputs of channels 8 n + w and 8 n + w + 4.  The
// partial logits meet in LDS (summed in wave order, so all four waves hold the
// same S and run the same softmax), and each wave writes its channels of the
// split's record.  At C2 a wave's page then takes about 60 % of the time.
constexpr int kSplitWaves = 4;
// Bytes of one logit-exchange buffer: every wave's S for RG row groups.
__host__ __device__ constexpr int xchg_bytes(int rg) { return kSplitWaves * rg * 2 * 4 * 64 * 4; }

// Every wave of the workgroup: this wave's LDS traffic done, then s_barrier.
// Outstanding page copies stay in flight.
__device__ __forceinline__ void block_lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Row groups of 4 query rows for GQ rows per KV head, and waves per workgroup:
// one-wave workgroups for 16 rows, whose LDS region (about 24 KB) leaves room
// for six waves per CU but not for two four-wave workgroups.
__host__ __device__ constexpr int fast_row_groups(int gq) { return gq > 4 ? gq / 4 : 1; }
__host__ __device__ constexpr int fast_waves_per_block(int gq) { return gq > 8 ? 1 : kWaves; }

// GQ: query rows per KV head (1, 2, 4, 8 or 16); NP: promoted channels (16,
// 32, 48 or 64); BF16: cache dtype bf16 (else fp16).  All compile-time, so
// every block loop unrolls with immediate offsets and the table builds carry
// no dtype tests.  Rows come in RG groups of GH: each group has its own Q K
// MFMAs (the slot layout holds 4 rows), with 8 or 16 rows the groups' A
// operands are formed per MFMA from one 2-byte LDS read each (several register
// sets would not fit; four reads per operand, three of zeros, stalled on LDS
// issue), as are the promoted pass's for any row count, and P V takes all rows
// in one MFMA (rows 4g + i: lane group kq = g holds group g's outputs).
//
// W: waves per split, 1 or kSplitWaves (channel-split pages, GQ <= 8).
template <int GQ, int NP, bool BF16, int W>
__global__ void __launch_bounds__(64 * fast_waves_per_block(GQ), 2)
    decode_pages_fast(FastParams p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15, kq = lane >> 4;
  static_assert(W == 1 || (W == kSplitWaves && fast_waves_per_block(GQ) == W), "one split per workgroup");
  const int mw = W > 1 ? wave : 0;  // this wave's quarter of a channel-split page
  const int total_workers = p.B * p.Hkv * p.splits;
  // page workers first (W waves each), then the dense-rest workers (one wave each)
  const int worker = W > 1 ? (int)blockIdx.x : (int)blockIdx.x * fast_waves_per_block(GQ) + wave;
  constexpr int np = NP;
  constexpr bool bf16 = BF16;
  constexpr int RG = fast_row_groups(GQ), GH = GQ > 4 ? 4 : GQ;
  static_assert(GQ == 1 || GQ == 2 || GQ == 4 || GQ == 8 || GQ == 16, "1, 2, 4, 8 or 16 query rows per KV head");
  const int gv = p.gv;
  const LdsMap M = lds_map(np, gv, RG);
  uint8_t* lds = smem + wave * M.bytes;
  if (worker >= total_workers) {  // a dense-rest worker, or none
    const int dw = W > 1 ? (worker - total_workers) * W + wave : worker - total_workers;
    dense_worker<GQ, BF16>(p, dw, lane, (float*)lds);
    return;
  }
  // wave-uniform indices (kept in scalar registers)
  const int split = __builtin_amdgcn_readfirstlane(worker % p.splits);
  const int bh = __builtin_amdgcn_readfirstlane(worker / p.splits);
  const int b = __builtin_amdgcn_readfirstlane(bh / p.Hkv), kvh = __builtin_amdgcn_readfirstlane(bh % p.Hkv);
  const int page0 = __builtin_amdgcn_readfirstlane((int)(((int64_t)split * p.count) / p.splits));
  const int page1 = __builtin_amdgcn_readfirstlane((int)(((int64_t)(split + 1) * p.count) / p.splits));

  // ---- per-lane constants ----
  const int sh = 2 * (n & 3);             // bit offset of this lane's codes in each byte
  const int qd = 8 * (n >> 2);            // byte offset of this lane's two code dwords in a 32-byte row
  const int slot = n >> 2, head = n & 3;  // slot-layout A row n = 4 * slot + head (row 4g + head of group g)
  // the non-zero A value's LDS address per row group (query and promoted
  // query), placed by slot_a; lanes of rows past GQ get zero operands
  const uint2 asel = slot_sel(slot, head < GH);
  int qsrc[RG], psrc[RG];
#pragma unroll
  for (int g = 0; g < RG; ++g) {
    qsrc[g] = M.q16 + 2 * ((4 * g + head) * kD + kq);
    psrc[g] = M.qp + kQpStride * (4 * g + head) + 2 * kq;
  }
  // P V A source (heads in rows): weights of head n, or zeros
  const int apv = n < GQ ? M.pt + kPtStride * n + 8 * kq : M.zero + 8 * kq;
  // P V block blk, K index 4kq + m is token 16 blk + kq + 4m: the four lane
  // groups then read code rows in different banks; the weights and the value
  // tables are stored in that K order (kpos), so each A operand is one 8-byte
  // read and a lane's four tables are one 32-byte run.
  const int vtab = M.vlut + kVlutStride * ((8 * n) / p.vg) + 32 * kq;  // value tables of the lane's group
  const int vcode = M.vc + 32 * kq + 2 * n;                           // value codes of the lane's channels

  // ---- running state ----
  // S (slot layout): lane (n, kq) holds rows 4g + 0..3 of tokens 32(n/4) + 16t + 4kq + n%4 in S[g][t].
  // O (rows in rows): lanes kq = g hold rows 4g + 0..3 of channels 8n + j in O[j].
  float m_run[RG][4], l_part[RG][4];
  float4v O[8 / W];  // channel-split waves: channels 8n + mw (O[0]) and 8n + mw + 4 (O[1])
#pragma unroll
  for (int g = 0; g < RG; ++g) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      m_run[g][i] = -INFINITY;
      l_part[g][i] = 0.f;
    }
  }
#pragma unroll
  for (int j = 0; j < 8 / W; ++j) O[j] = float4v{0.f, 0.f, 0.f, 0.f};

  int qexp;  // the query's power-of-two scale (query_exponent)
  {
    uint16_t* q16 = (uint16_t*)(lds + M.q16);
    float qv[4 * RG * kD / 64];
    dev_load_n(p.query, p.q_dtype, qv, [&](int r) -> int64_t {
      const int i = lane + 64 * r, h = i / kD, c = i % kD;
      return h < GQ ? (int64_t)b * p.q_sb + (int64_t)(kvh * GQ + h) * p.q_sh + c : -1;
    });
    qexp = query_exponent(qv);
#pragma unroll
    for (int r = 0; r < 4 * RG * kD / 64; ++r)
      q16[lane + 64 * r] = __builtin_bit_cast(uint16_t, (_Float16)ldexpf(qv[r], -qexp));
    *(uint32_t*)(lds + M.zero + 4 * lane) = 0u;
  }
  lds_sync();
  // Q K A operands for channel blocks cb = 0..31 (natural channel order), kept
  // in registers for the whole split: q[head][4cb + kq] at half `slot` (with
  // one row group; with two they are read from q16 per MFMA, qsrc).
  // (a channel-split wave keeps its own blocks cb0 .. cb0 + kD / 4 / W - 1)
  const int cb0 = kD / 4 / W * mw;
  half4 qa[RG == 1 ? kD / 4 / W : 1];
  if constexpr (RG == 1) {
    const uint16_t* q16 = (const uint16_t*)(lds + M.q16);
#pragma unroll
    for (int cb = 0; cb < kD / 4 / W; ++cb) {
      const _Float16 v = __builtin_bit_cast(_Float16, q16[head * kD + 4 * (cb0 + cb) + kq]);
#pragma unroll
      for (int i = 0; i < 4; ++i) qa[cb][i] = i == slot ? v : (_Float16)0.f;
    }
  }
  if (page0 < page1) {
    const PageAddr a0 = page_addr(descriptor(p.segs, p.first + page0), bh);
    issue_small(M, lds, a0, np, gv, lane);
    issue_keys(M, lds, a0, np, lane);
    issue_values(M, lds, a0, lane);
  }
  const float c2 = ldexpf(p.scale * kLog2e, qexp);
  const uint32_t m3 = in_sgpr(0x03030303u);
  const uint32_t sel2 = in_vgpr(0x04000400u);
  // LDS address of the 4-bit tables; its low byte is zero (the map and every
  // wave's region are 256-aligned and the dynamic LDS starts at 0).  Were it
  // not, the split's records are poisoned (NaN) rather than wrong.
  const uint32_t tab16 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void*)(lds + M.klut16));

#pragma unroll 1
  for (int pg = page0; pg < page1; ++pg) {
    const bool has_next = pg + 1 < page1;
    PageAddr nxt;
    if (has_next) nxt = page_addr(descriptor(p.segs, p.first + pg + 1), bh);
    // outstanding, oldest first: scales (this page), key codes (this page),
    // value codes (this page, 4 loads); the values may still be in flight
    vm_wait(4);

    // ---- 2-bit key tables of every channel, and a byte-wide copy of the
    // promoted channels (the index region is refilled early) ----
    uint8_t* pidx = lds + M.pidx;
    const uint16_t* ks = (const uint16_t*)(lds + M.ks);
    const uint16_t* kz = (const uint16_t*)(lds + M.kz);
    int my_promoted = 0;
    if (lane < np) {
      my_promoted = ((const int32_t*)(lds + M.ki))[lane] & 127;
      pidx[lane] = (uint8_t)my_promoted;
    }
#pragma unroll
    for (int c = lane; c < kD; c += 64) *(uint2*)(lds + M.klut + 8 * key_slot(c)) = build_lut4<bf16>(ks[c], kz[c]);
    lds_sync();
    // promoted channels take the 4-bit pass: their 2-bit tables become zero
    if (lane < np) *(uint2*)(lds + M.klut + 8 * key_slot(my_promoted)) = make_uint2(0u, 0u);
    lds_sync();

    // ---- S = Q K; tile t covers tokens 32(n/4) + 16t + 4 slot + n%4 ----
    float4v S[RG][2];
#pragma unroll
    for (int g = 0; g < RG; ++g) S[g][0] = S[g][1] = float4v{0.f, 0.f, 0.f, 0.f};
    // 2-bit codes of every channel (promoted channels have zero tables), one
    // pair of channel blocks (2u, 2u + 1) per step: each block's code dwords of
    // both tiles are one 8-byte read and the pair's tables one 16-byte read;
    // pair u + 1's are read before pair u is computed.  The tables the later
    // passes need (value tables, 4-bit key tables, the promoted channels'
    // query) are built in between, so their LDS latency overlaps the lookups.
    {
      // a channel-split wave takes pairs u0 .. u0 + NU - 1 (its qa blocks)
      constexpr int NU = kD / 8 / W;
      const int u0 = NU * mw;
      const int row = M.kl + 32 * kq + qd + 256 * u0;
      const int tab = M.klut + 16 * kq + 64 * u0;
      const uint16_t* vs = (const uint16_t*)(lds + M.vs);
      const uint16_t* vz = (const uint16_t*)(lds + M.vz);
      if constexpr (W > 1) {
        // every table, before this wave's share of the lookups
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int tt = lane + 64 * (k & 1), g = (k >> 1) % gv;
          *(uint2*)(lds + M.vlut + kVlutStride * g + 8 * kpos(tt)) = build_lut4<bf16>(vs[tt * gv + g], vz[tt * gv + g]);
        }
        build_lut16_tables<bf16, np>(M, lds, ks, kz, lane);
        const uint16_t* q16 = (const uint16_t*)(lds + M.q16);
        const uint8_t* pidx = lds + M.pidx;
        uint16_t* qp = (uint16_t*)(lds + M.qp);
#pragma unroll
        for (int i = lane; i < GQ * np; i += 64) {
          const int h = i / np, j = i % np;
          qp[h * (kQpStride / 2) + j] = q16[h * kD + pidx[j]];
        }
      }
      uint2 wc[2 * NU];
      uint4 t[NU];
      auto load_pair = [&](int u) {
        wc[2 * u] = *(const uint2*)(lds + row + 256 * u);
        wc[2 * u + 1] = *(const uint2*)(lds + row + 256 * u + 128);
        t[u] = *(const uint4*)(lds + tab + 64 * u);
      };
      load_pair(0);
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        if (u + 1 < NU) load_pair(u + 1);
        const half4 b0e = lookup4((wc[2 * u].x >> sh) & 0x03030303u, t[u].x, t[u].y);
        const half4 b1e = lookup4((wc[2 * u].y >> sh) & 0x03030303u, t[u].x, t[u].y);
        const half4 b0o = lookup4((wc[2 * u + 1].x >> sh) & 0x03030303u, t[u].z, t[u].w);
        const half4 b1o = lookup4((wc[2 * u + 1].y >> sh) & 0x03030303u, t[u].z, t[u].w);
        if constexpr (RG == 1) {
          S[0][0] = mma2(qa[2 * u], qa[2 * u + 1], b0e, b0o, S[0][0]);
          S[0][1] = mma2(qa[2 * u], qa[2 * u + 1], b1e, b1o, S[0][1]);
        } else {
#pragma unroll
          for (int g = 0; g < RG; ++g) {
            const half4 a0 = slot_a(*(const uint16_t*)(lds + qsrc[g] + 16 * (u0 + u)), asel);
            const half4 a1 = slot_a(*(const uint16_t*)(lds + qsrc[g] + 16 * (u0 + u) + 8), asel);
            S[g][0] = mma2(a0, a1, b0e, b0o, S[g][0]);
            S[g][1] = mma2(a0, a1, b1e, b1o, S[g][1]);
          }
        }
        if (W == 1 && u % 2 == 0 && u / 2 < 4) {
          // value table k = u / 2 of this lane: token lane + 64 (k & 1), group k >> 1
          // (groups beyond gv rebuild an existing table with identical contents)
          const int k = u / 2;
          const int tt = lane + 64 * (k & 1), g = (k >> 1) % gv;
          *(uint2*)(lds + M.vlut + kVlutStride * g + 8 * kpos(tt)) = build_lut4<bf16>(vs[tt * gv + g], vz[tt * gv + g]);
        }
        if (W == 1 && u == 9) build_lut16_tables<bf16, np>(M, lds, ks, kz, lane);
        if (W == 1 && u == 13) {
          const uint16_t* q16 = (const uint16_t*)(lds + M.q16);
          const uint8_t* pidx = lds + M.pidx;
          uint16_t* qp = (uint16_t*)(lds + M.qp);
#pragma unroll
          for (int i = lane; i < GQ * np; i += 64) {
            const int h = i / np, j = i % np;
            qp[h * (kQpStride / 2) + j] = q16[h * kD + pidx[j]];
          }
        }
      }
    }
    // value tables of groups 2.. (value groups narrower than 64 channels)
    for (int i = 256 + lane; i < kPage * gv; i += 64) {
      const int g = i >> 7, tt = i & 127;
      const uint16_t* vs = (const uint16_t*)(lds + M.vs);
      const uint16_t* vz = (const uint16_t*)(lds + M.vz);
      *(uint2*)(lds + M.vlut + kVlutStride * g + 8 * kpos(tt)) = build_lut4<bf16>(vs[tt * gv + g], vz[tt * gv + g]);
    }
    lds_sync();
    // promoted channels: 4-bit codes, slot j = 4pb + kq of the high codes;
    // block pb + 1's codes and tables are read before block pb is computed
    {
      const uint32_t rl = (uint32_t)(sh - 1) & 31u, rh = (uint32_t)(sh - 3) & 31u;
      const uint32_t kq32 = 0x20202020u * (uint32_t)kq;
      const uint32_t m6 = in_sgpr(0x06060606u), m18 = in_sgpr(0x18181818u);
      if constexpr (W > 1) {
        // block pairs (2 pp, 2 pp + 1) for pp = mw, mw + W, ...: the pair's
        // tables start at tab16 + 256 pp (low byte still zero), the odd
        // block's 128 bytes on
        constexpr int NPP = np / 8;
#pragma unroll
        for (int i = 0; i < (NPP + W - 1) / W; ++i) {
          const int pp = mw + W * i;
          if (pp < NPP) {
            uint2 wlp[2], whp[2];
            half4 ap[2][RG];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
              const int j = 4 * (2 * pp + e) + kq;
              wlp[e] = *(const uint2*)(lds + M.kl + 32 * pidx[j] + qd);
              whp[e] = *(const uint2*)(lds + M.kh + 32 * j + qd);
#pragma unroll
              for (int g = 0; g < RG; ++g) ap[e][g] = slot_a(*(const uint16_t*)(lds + psrc[g] + 8 * (2 * pp + e)), asel);
            }
            const uint32_t tabp = tab16 + 256u * (uint32_t)pp;
            const half4 b00 = gather16(wlp[0].x, whp[0].x, rl, rh, kq32, tabp, 0, m6, m18);
            const half4 b01 = gather16(wlp[0].y, whp[0].y, rl, rh, kq32, tabp, 0, m6, m18);
            const half4 b10 = gather16(wlp[1].x, whp[1].x, rl, rh, kq32, tabp, 128, m6, m18);
            const half4 b11 = gather16(wlp[1].y, whp[1].y, rl, rh, kq32, tabp, 128, m6, m18);
#pragma unroll
            for (int g = 0; g < RG; ++g) {
              S[g][0] = mma2(ap[0][g], ap[1][g], b00, b10, S[g][0]);
              S[g][1] = mma2(ap[0][g], ap[1][g], b01, b11, S[g][1]);
            }
          }
        }
      } else {
      uint2 wl[np / 4], wh[np / 4];  // .x: tile 0, .y: tile 1
      auto load_pb = [&](int pb) {
        const int j = 4 * pb + kq;
        wl[pb] = *(const uint2*)(lds + M.kl + 32 * pidx[j] + qd);
        wh[pb] = *(const uint2*)(lds + M.kh + 32 * j + qd);
      };
      load_pb(0);
      half4 pa[RG], pend0, pend1;  // even block's operands, waiting for the odd one (np / 4 is even)
#pragma unroll
      for (int pb = 0; pb < np / 4; ++pb) {
        if (pb + 1 < np / 4) load_pb(pb + 1);
        half4 a[RG];
#pragma unroll
        for (int g = 0; g < RG; ++g) a[g] = slot_a(*(const uint16_t*)(lds + psrc[g] + 8 * pb), asel);
        const half4 b0 = gather16(wl[pb].x, wh[pb].x, rl, rh, kq32, tab16, 128 * pb, m6, m18);
        const half4 b1 = gather16(wl[pb].y, wh[pb].y, rl, rh, kq32, tab16, 128 * pb, m6, m18);
        if (pb & 1) {
#pragma unroll
          for (int g = 0; g < RG; ++g) {
            S[g][0] = mma2(pa[g], a[g], pend0, b0, S[g][0]);
            S[g][1] = mma2(pa[g], a[g], pend1, b1, S[g][1]);
          }
        } else {
#pragma unroll
          for (int g = 0; g < RG; ++g) pa[g] = a[g];
          pend0 = b0;
          pend1 = b1;
        }
      }
      }
    }
    lds_sync();
    if constexpr (W > 1) {
      // the waves' partial logits, summed in wave order (two buffers by page
      // parity: a wave one page ahead writes the other one)
      float* xs = (float*)(smem + kSplitWaves * M.bytes + xchg_bytes(RG) * (pg & 1));
#pragma unroll
      for (int g = 0; g < RG; ++g)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) xs[(((mw * RG + g) * 2 + t) * 4 + i) * 64 + lane] = S[g][t][i];
      block_lds_barrier();
#pragma unroll
      for (int g = 0; g < RG; ++g)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float acc = xs[((g * 2 + t) * 4 + i) * 64 + lane];
#pragma unroll
            for (int w = 1; w < W; ++w) acc += xs[(((w * RG + g) * 2 + t) * 4 + i) * 64 + lane];
            S[g][t][i] = acc;
          }
    }
    if (has_next) {
      issue_small(M, lds, nxt, np, gv, lane);
      issue_keys(M, lds, nxt, np, lane);
    }

    // ---- online softmax in base 2 ----
    {
      float x[RG][2][4];
      bool over = false;
#pragma unroll
      for (int g = 0; g < RG; ++g) {
#pragma unroll
        for (int i = 0; i < GH; ++i) {
          x[g][0][i] = S[g][0][i] * c2;
          x[g][1][i] = S[g][1][i] * c2;
          over |= fmaxf(x[g][0][i], x[g][1][i]) > m_run[g][i] + kSlack;
        }
      }
      if (__ballot(over) != 0ull) {
        float alpha[RG][4];
#pragma unroll
        for (int g = 0; g < RG; ++g) {
#pragma unroll
          for (int i = 0; i < GH; ++i) {
            const float m_new = uniform(fmaxf(m_run[g][i], wave_max64(fmaxf(x[g][0][i], x[g][1][i]))));
            alpha[g][i] = __builtin_amdgcn_exp2f(m_run[g][i] - m_new);
            l_part[g][i] *= alpha[g][i];
            m_run[g][i] = m_new;
          }
        }
#pragma unroll
        for (int i = 0; i < GH; ++i) {
          // O row 4g + i sits in lane group kq = g (rows past GQ are zero)
          float al = alpha[0][i];
#pragma unroll
          for (int g = 1; g < RG; ++g) al = kq == g ? alpha[g][i] : al;
#pragma unroll
          for (int j = 0; j < 8 / W; ++j) O[j][i] *= al;
        }
      }
      uint16_t* pt = (uint16_t*)(lds + M.pt);
      const int tok = 32 * (n >> 2) + 4 * kq + (n & 3);  // tile 0; tile 1 is tok + 16
      const int wpos = kpos(tok);
#pragma unroll
      for (int g = 0; g < RG; ++g) {
#pragma unroll
        for (int i = 0; i < GH; ++i) {
          const float p0 = __builtin_amdgcn_exp2f(x[g][0][i] - m_run[g][i]);
          const float p1 = __builtin_amdgcn_exp2f(x[g][1][i] - m_run[g][i]);
          l_part[g][i] += p0 + p1;
          pt[(4 * g + i) * (kPtStride / 2) + wpos] = __builtin_bit_cast(uint16_t, (_Float16)p0);
          pt[(4 * g + i) * (kPtStride / 2) + wpos + 16] = __builtin_bit_cast(uint16_t, (_Float16)p1);
        }
      }
    }
    lds_sync();

    // this page's value codes are older than the next page's scale and key
    // loads issued since
    vm_wait(has_next ? n_small_loads(np, gv) + n_key_loads(np) : 0);

    // ---- O += P V, heads in rows: block blk covers tokens 16 blk + kq + 4m ----
    // (block blk + 1's weights, codes and tables are read before block blk is computed)
    {
      half4 a[kPage / 16];
      uint32_t x[kPage / 16][4], lo[kPage / 16][4], hi[kPage / 16][4];
      auto load_blk = [&](int blk) {
        a[blk] = *(const half4*)(lds + apv + 32 * blk);
#pragma unroll
        for (int m = 0; m < 4; ++m) x[blk][m] = *(const uint16_t*)(lds + vcode + 512 * blk + 128 * m);
        const uint4 t01 = *(const uint4*)(lds + vtab + 128 * blk);
        const uint4 t23 = *(const uint4*)(lds + vtab + 128 * blk + 16);
        lo[blk][0] = t01.x; hi[blk][0] = t01.y; lo[blk][1] = t01.z; hi[blk][1] = t01.w;
        lo[blk][2] = t23.x; hi[blk][2] = t23.y; lo[blk][3] = t23.z; hi[blk][3] = t23.w;
      };
      load_blk(0);
      uint2 wprev[8 / W];  // even block's B operands, waiting for the odd one
#pragma unroll
      for (int blk = 0; blk < kPage / 16; ++blk) {
        if (blk + 1 < kPage / 16) load_blk(blk + 1);
        uint2 wk[8 / W];
        lut_block_operands<W>(x[blk], lo[blk], hi[blk], wk, m3, sel2, mw);
        if (blk & 1) {
#pragma unroll
          for (int j = 0; j < 8 / W; ++j)
            O[j] = mma2(a[blk - 1], a[blk], __builtin_bit_cast(half4, wprev[j]), __builtin_bit_cast(half4, wk[j]),
                        O[j]);
        } else {
#pragma unroll
          for (int j = 0; j < 8 / W; ++j) wprev[j] = wk[j];
        }
      }
    }
    lds_sync();
    if (has_next) issue_values(M, lds, nxt, lane);
  }

  // ---- partial state ----
#pragma unroll
  for (int g = 0; g < RG; ++g) {
#pragma unroll
    for (int i = 0; i < GH; ++i) {
      const float l = wave_sum64(l_part[g][i]);
      const int hq = kvh * GQ + 4 * g + i;
      float* rec = p.ws + (((int64_t)b * p.Hq + hq) * p.split_stride + split) * (kD + 2);
      if (lane == 0 && mw == 0) {
        rec[0] = (tab16 & 255u) == 0 ? m_run[g][i] * kLn2 : NAN;
        rec[1] = l;
      }
      if (kq == g) {
        if constexpr (W == 1) {
#pragma unroll
          for (int j = 0; j < 8; ++j) rec[2 + 8 * n + j] = O[j][i];
        } else {
          rec[2 + 8 * n + mw] = O[0][i];
          rec[6 + 8 * n + mw] = O[1][i];
        }
      }
    }
  }
}

}  // namespace

namespace dkv {

int fast_decode_max_loads(int np, int gv) { return n_small_loads(np, gv) + n_key_loads(np); }

size_t fast_decode_lds_bytes(int np, int gv, int gq) {
  return (size_t)fast_waves_per_block(gq) * lds_map(np, gv, fast_row_groups(gq)).bytes;
}

// Compute units of the current device (read once per device; threads that
// race on the first read store the same value).
static int device_cus() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cus[kMaxDevices] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

int launch_fast_decode(const dkv_decode_args& a, int first, int count, int np, int vg, int splits, int split_stride,
                       hipStream_t stream, const FusedRest* fused) {
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
  set_fused(p, fused);
  const int64_t page_workers = (int64_t)p.B * p.Hkv * splits;
  const int wpb = fast_waves_per_block(p.GQ);
  // Channel-split pages when every workgroup of that launch (one split each,
  // then the dense-rest waves four to a workgroup) has a compute unit to
  // itself: the launch leaves most of the GPU idle, and a page's latency
  // bounds the call.  DKV_SPLIT_PAGES=0 / 1 in the environment turns them off
  // / on for every launch that can take them (tests compare the two).
  const int64_t split_blocks = page_workers + (p.dense_workers + kSplitWaves - 1) / kSplitWaves;
  const char* force = getenv("DKV_SPLIT_PAGES");
  bool split_pages = false;
  if (wpb == kSplitWaves) {
    if (force != nullptr && force[0] != '\0') {
      split_pages = force[0] != '0';
    } else {
      const int cus = device_cus();
      split_pages = cus > 0 && split_blocks <= cus;
    }
  }
  const unsigned blocks =
      (unsigned)(split_pages ? split_blocks : (page_workers + p.dense_workers + wpb - 1) / wpb);
  const size_t lds = fast_decode_lds_bytes(np, p.gv, p.GQ) +
                     (split_pages ? (size_t)2 * xchg_bytes(fast_row_groups(p.GQ)) : 0);
  const dim3 grid(blocks), block(64 * wpb);
#define DKV_FAST_LAUNCH(G, N)                                                                             \
  do {                                                                                                    \
    if (split_pages && G <= 8) {                                                                          \
      if (p.bf16) hipLaunchKernelGGL((decode_pages_fast<G, N, true, G <= 8 ? kSplitWaves : 1>), grid, block, lds, stream, p); \
      else hipLaunchKernelGGL((decode_pages_fast<G, N, false, G <= 8 ? kSplitWaves : 1>), grid, block, lds, stream, p);      \
    } else {                                                                                              \
      if (p.bf16) hipLaunchKernelGGL((decode_pages_fast<G, N, true, 1>), grid, block, lds, stream, p);    \
      else hipLaunchKernelGGL((decode_pages_fast<G, N, false, 1>), grid, block, lds, stream, p);          \
    }                                                                                                     \
  } while (0)
#define DKV_FAST_NP(G)                         \
  switch (np) {                                \
    case 16: DKV_FAST_LAUNCH(G, 16); break;    \
    case 32: DKV_FAST_LAUNCH(G, 32); break;    \
    case 48: DKV_FAST_LAUNCH(G, 48); break;    \
    default: DKV_FAST_LAUNCH(G, 64); break;    \
  }
  if (np != 16 && np != 32 && np != 48 && np != 64) {
    set_error("fast decode supports 16, 32, 48 or 64 promoted channels");
    return DKV_ERR_UNSUPPORTED;
  }
  switch (p.GQ) {
    case 1: DKV_FAST_NP(1); break;
    case 2: DKV_FAST_NP(2); break;
    case 4: DKV_FAST_NP(4); break;
    case 8: DKV_FAST_NP(8); break;
    case 16: DKV_FAST_NP(16); break;
    default:
      set_error("fast decode supports 1, 2, 4, 8 or 16 query rows per KV head");
      return DKV_ERR_UNSUPPORTED;
  }
#undef DKV_FAST_NP
#undef DKV_FAST_LAUNCH
  return dkv_check_launch("dkv_decode_attention(fast pages)");
}

}  // namespace dkv
