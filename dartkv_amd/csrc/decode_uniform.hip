// Single-token decode over full uniform pages (gfx950, wave64).
//
// Scope: head_dim 128, 128-token pages, keys quantized uniformly with KB bits
// along the tokens (one key group per page), values with VB bits along the
// channels in groups of vg (16 | vg, vg | 128), KB, VB in {2, 4, 8}, fp16
// metadata, bf16 or fp16 cache, 1, 2, 4 or 8 query rows per KV head (8: two
// row groups of 4, each with its own Q K and P V MFMAs on the same
// dequantized operands, the A operands formed from one LDS read each).
//
// Each wave owns a split: a contiguous range of half pages (64 tokens; half
// page q is half q & 1 of page q >> 1) of one (batch, kv head).  It stages a
// page's key codes (every channel) and key scales once, when the page starts
// (for 8-bit keys, whose LDS would double, each half stages its own half of
// every key row), and each half's value rows and scales; then per half page
//   * S = Q K with MFMAs in the slot layout (rows = 4 slots x
//     4 query heads; a lane's four B values are four tokens of one channel,
//     A carries the query at the lane's slot); one tile covers the 64 tokens;
//   * an online softmax in base 2 (running max moves only beyond 8);
//   * O += P V in the same slot layout (a lane's four B values are four
//     channels of one token; A carries the weight at the lane's slot), two
//     tiles of 64 channels.
// 2- and 4-bit codes are dequantized by exact-value tables (with 1, 2 or 4
// query rows; for values, with value groups of 64 or 128 channels): every key
// channel's table (its 2^B values under the reference's rounding chain,
// fp16(fp16(code * scale) + zero) and, for bf16 caches, bf16 precision) is
// built once per page and every (token, value group)'s once per quarter page;
// a B operand is then four 2-byte LDS gathers.  Each lane group of 16 reads
// one 32-byte table (8 banks) and the four groups' tables sit in distinct
// banks, so the gathers do not conflict.  Otherwise codes are dequantized
// arithmetically with the same rounding chain: codes below 16 become fp16
// through the fp8 converter (the e4m3 pattern of a code c < 16 is c * 2^-9:
// subnormals and the first binade are evenly spaced, and the converter's
// power-of-two scale 2^9 restores c), 8-bit codes through byte permutes
// under the fp16 exponent of 1024 (0x64xx = 1024 + code) less 1024, with
// scales and zero points duplicated into (s, s, z, z) tables once per page
// (keys) or half (values).
#include <hip/hip_runtime.h>
#include <math.h>

#include "dkv_capi_util.h"
#include "dkv_decode.h"
#include "dkv_device.h"
#include "dkv_page_common.h"

using namespace dkv;

namespace {

constexpr int kHalfTok = 64;   // tokens per half page
constexpr int kPtRow = 160;    // bytes between softmax-weight rows ([4][64] fp16, 8 banks apart)

struct UMap {
  int kc, vc, ks, kz, vs, vz, kt, vt, q16, pt, zero, bytes;
};

// Exact-value tables (32 bytes each, 2^B fp16 entries) for B-bit keys with
// 1, 2 or 4 query rows, and for B-bit values as well when their groups are
// 64 or 128 channels wide (at most two per token, so a quarter page's tables
// fit beside the rest of the wave's LDS).
__host__ __device__ constexpr bool key_tables(int kb, int gq) { return kb <= 4 && gq <= 4; }
__host__ __device__ constexpr bool value_tables_ok(int vb, int gq) { return vb <= 4 && gq <= 4; }
constexpr int kTable = 32;      // bytes per table
constexpr int kQuarterTok = 32; // tokens whose value tables are built at a time

// Key rows staged per page (2: both halves of every channel's 16 KB-byte row)
// or per half page (1).  A half row is half a 128-byte line for 2- and 4-bit
// keys; staging it per half would fetch the line again once L2 has dropped it.
__host__ __device__ constexpr int key_rows_per_stage(int kb) { return kb <= 4 ? 2 : 1; }

// rg: row groups of 4 query rows (the query and the softmax weights take 4 rg
// rows); kt / vt: key / value tables (else (s, s, z, z) entries).  Tables
// start on a 256-byte boundary (gather4 forms addresses by byte permutes) and
// so does every wave's region when there are any.
__host__ __device__ inline UMap umap(int kb, int vb, int gv, int rg, bool kt, bool vt) {
  UMap m;
  int o = 0;
  const int kf = key_rows_per_stage(kb);
  m.kc = o; o += kD * 8 * kb * kf;     // key codes [128 ch][8 KB kf bytes]
  m.vc = o; o += kHalfTok * 16 * vb;   // value codes of the half [64 tok][16 VB bytes]
  m.ks = o; o += 256;                  // key scale [128] fp16
  m.kz = o; o += 256;                  // key zero  [128] fp16
  m.vs = o; o += 128 * gv;             // value scale of the half [64 tok][Gv] fp16
  m.vz = o; o += 128 * gv;             // value zero  of the half [64 tok][Gv] fp16
  if (kt) {
    o = (o + 255) / 256 * 256;
    m.kt = o; o += kD * kTable;        // key tables [128 ch][2^KB] fp16
  } else {
    m.kt = o; o += kD * 8;             // key (s, s, z, z) per channel [128] (fp16 pairs)
  }
  if (vt) {
    o = (o + 255) / 256 * 256;
    m.vt = o; o += gv * kQuarterTok * kTable;  // value tables of a quarter page [Gv][32 tok][2^VB] fp16
  } else {
    m.vt = o; o += kHalfTok * 8 * gv;  // value (s, s, z, z) of the half [64 tok][Gv]
  }
  if (vt && rg == 1 && gv * kQuarterTok * kTable >= 1024) {
    m.q16 = m.vt;                      // the query is read once, before any value table is built
  } else {
    m.q16 = o; o += 1024 * rg;         // query [4 rg][128 ch] fp16 (split start only, and per MFMA with 2 groups)
  }
  o = (o + 127) / 128 * 128;
  m.pt = o; o += 4 * rg * kPtRow;      // softmax weights [4 rg][64 tok] fp16
  o = (o + 127) / 128 * 128 + 64;
  m.zero = o; o += 256;                // zeros read by A-operand lanes without data
  m.bytes = (kt || vt) ? (o + 255) / 256 * 256 : (o + 15) / 16 * 16;
  return m;
}

// Staging: key scales and codes of a page (or half page, see above), issued
// after the Q K of the half before it, then value codes and value scales of a
// half page (issued after the P V of the half before it).
// The scales and zero points of a stage share copies: each lane of a copy
// reads its own 16 bytes, so one copy fills the adjacent scale and zero
// regions (M.kz = M.ks + 256, M.vz = M.vs + 128 gv).
__host__ __device__ inline int n_key_loads_u(int kb) { return kb * key_rows_per_stage(kb) + 1; }
__host__ __device__ inline int n_value_loads_u(int vb, int gv) { return vb + (16 * gv + 63) / 64; }

__device__ __forceinline__ void issue_keys_u(const UMap& M, uint8_t* lds, const PageAddr& a, int kb, int h,
                                             int lane) {
  {
    const uint32_t dst = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void*)(lds + M.ks));
    const int64_t to_kz = byte_gap(a.kz, a.ks) - 256;
    if (lane < 32) dma16(byte_at(a.ks, 16 * lane + (lane >= 16 ? to_kz : 0)), dst);
  }
  const int kf = key_rows_per_stage(kb);
  if (kf == 2) {  // whole rows: one contiguous block
    copy_to_lds(lds + M.kc, a.kl, kD * 16 * kb, lane);
    return;
  }
  // 16-byte chunk i of the half's codes: row i / cpr, column i % cpr
  const int cpr = kb / 2;
  const uint32_t base = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void*)(lds + M.kc));
  for (int i0 = 0; i0 < kD * cpr; i0 += 64) {
    const int i = i0 + lane, row = i / cpr, col = i % cpr;
    dma16(a.kl + 16 * kb * row + 8 * kb * h + 16 * col, base + 16 * i0);
  }
}
__device__ __forceinline__ void issue_values_u(const UMap& M, uint8_t* lds, const PageAddr& a, int vb, int gv, int h,
                                               int lane) {
  copy_to_lds(lds + M.vc, a.vc + 16 * vb * kHalfTok * h, 16 * vb * kHalfTok, lane);
  const uint32_t dst = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void*)(lds + M.vs));
  const int64_t to_vz = byte_gap(a.vz, a.vs) - 128 * gv;  // the half's zero points follow its scales
  for (int off = 0; off < 256 * gv; off += 1024) {
    const int i = (off >> 4) + lane;
    if (i < 16 * gv) dma16(byte_at(a.vs, 128 * gv * h + 16 * i + (i >= 8 * gv ? to_vz : 0)), dst + off);
  }
}

// Four codes (one per byte of e, values 0..2^B - 1) -> their dequantized
// values as an fp16 B operand: fp16(fp16(code * s) + z), bf16 precision if
// BF16.  sz holds (s, s) and (z, z); the ops stay separate (-ffp-contract=off).
template <int B, bool BF16>
__device__ __forceinline__ half4 dequant4(uint32_t e, uint2 sz) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 s = __builtin_bit_cast(h2, sz.x), z = __builtin_bit_cast(h2, sz.y);
  h2 c01, c23;  // codes 0, 1 and 2, 3
  if (B <= 4) {
    c01 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(e, 512.f, false);
    c23 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(e, 512.f, true);
  } else {
    const h2 off = {(_Float16)-1024.f, (_Float16)-1024.f};
    c01 = __builtin_bit_cast(h2, perm(0x64646464u, e, 0x04010400u)) + off;
    c23 = __builtin_bit_cast(h2, perm(0x64646464u, e, 0x04030402u)) + off;
  }
  const h2 p01 = c01 * s, p23 = c23 * s;
  uint32_t v01 = __builtin_bit_cast(uint32_t, p01 + z), v23 = __builtin_bit_cast(uint32_t, p23 + z);
  if (BF16) {
    v01 = round_pair_to_bf16_precision(v01);
    v23 = round_pair_to_bf16_precision(v23);
  }
  return __builtin_bit_cast(half4, make_uint2(v01, v23));
}

// Lane n's position in a dword of B-bit codes: tpb = 8 / B codes per byte;
// the lane reads dword n / tpb of a row and takes bit field n % tpb of each of
// its 4 bytes, i.e. codes 4 tpb (n / tpb) + tpb j + n % tpb, j = 0..3.
template <int B>
__device__ __forceinline__ int code_index(int n, int j) {
  constexpr int tpb = 8 / B;
  return 4 * tpb * (n / tpb) + tpb * j + n % tpb;
}
template <int B>
__device__ __forceinline__ uint32_t code_mask() {
  return B == 8 ? 0xffffffffu : (B == 4 ? 0x0f0f0f0fu : 0x03030303u);
}

// (s, s, z, z) table entries from fp16 scale / zero arrays: lanes take
// entries lane, lane + 64, ... of n.
__device__ __forceinline__ void build_sz_table(uint8_t* lds, int dst, int src_s, int src_z, int n, int lane) {
  const uint16_t* s = (const uint16_t*)(lds + src_s);
  const uint16_t* z = (const uint16_t*)(lds + src_z);
  for (int i = lane; i < n; i += 64)
    *(uint2*)(lds + dst + 8 * i) = make_uint2((uint32_t)s[i] * 0x10001u, (uint32_t)z[i] * 0x10001u);
}

// Half h of the exact-value table of one (scale, zero) pair: codes
// h 2^(B-1) .. (h + 1) 2^(B-1) - 1 (B = 2 or 4), written at dst.
template <int B, bool BF16>
__device__ __forceinline__ void build_table_half(uint8_t* lds, int dst, uint16_t s, uint16_t z, int h) {
  const half2v s2 = splat_h(s), z2 = splat_h(z);
  if constexpr (B == 4) {
    uint32_t v[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = lut_pair<BF16>(code_pair(q, h), s2, z2);
    *(uint4*)(lds + dst + 16 * h) = make_uint4(v[0], v[1], v[2], v[3]);
  } else {
    *(uint32_t*)(lds + dst + 4 * h) = lut_pair<BF16>(code_pair(h, 0), s2, z2);  // codes (2h, 2h + 1)
  }
}

// Key tables of a page: channel c's at kt + 32 c; item i is half i & 1 of channel i >> 1.
template <int B, bool BF16>
__device__ __forceinline__ void build_key_tables(const UMap& M, uint8_t* lds, int lane) {
  const uint16_t* ks = (const uint16_t*)(lds + M.ks);
  const uint16_t* kz = (const uint16_t*)(lds + M.kz);
#pragma unroll
  for (int i = lane; i < 2 * kD; i += 64) build_table_half<B, BF16>(lds, M.kt + kTable * (i >> 1), ks[i >> 1], kz[i >> 1], i & 1);
}

// Value tables of quarter page qr of the half: (token 32 qr + t, group g)'s
// at vt + 1024 g + 32 t; item i is half i & 1 of table i >> 1 = 32 g + t.
template <int B, bool BF16>
__device__ __forceinline__ void build_value_tables(const UMap& M, uint8_t* lds, int gv, int qr, int lane) {
  const uint16_t* vs = (const uint16_t*)(lds + M.vs);
  const uint16_t* vz = (const uint16_t*)(lds + M.vz);
  for (int i = lane; i < 2 * kQuarterTok * gv; i += 64) {
    const int g = i >> 6, t = (i >> 1) & 31, src = (kQuarterTok * qr + t) * gv + g;
    build_table_half<B, BF16>(lds, M.vt + kQuarterTok * kTable * g + kTable * t, vs[src], vz[src], i & 1);
  }
}

// Byte j of the result = 2 x the B-bit code at bits [shift + 8 j, shift + 8 j + B)
// of w, plus add (rot = (shift - 1) mod 32).
template <int B>
__device__ __forceinline__ uint32_t twice_code_bytes(uint32_t w, uint32_t rot, uint32_t add) {
  const uint32_t mask = B == 4 ? 0x1e1e1e1eu : 0x06060606u;
  return (__builtin_amdgcn_alignbit(w, w, rot) & mask) | add;
}

template <int GQ, int KB, int VB, bool BF16, bool VTAB>
__global__ void __launch_bounds__(256) decode_pages_uniform(FastParams p) {
  constexpr int RG = GQ > 4 ? 2 : 1, GH = GQ > 4 ? 4 : GQ;  // row groups of GH query rows
  static_assert(GQ == 1 || GQ == 2 || GQ == 4 || GQ == 8, "1, 2, 4 or 8 query rows per KV head");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15, kq = lane >> 4;
  const int worker = blockIdx.x * kWaves + wave;
  constexpr bool KT = key_tables(KB, GQ), VT = VTAB;  // exact-value tables for keys / values
  static_assert(!VT || value_tables_ok(VB, GQ), "value tables need 2- or 4-bit values and at most 4 query rows");
  const int gv = p.gv;
  const UMap M = umap(KB, VB, gv, RG, KT, VT);
  uint8_t* lds = smem + wave * M.bytes;
  if (worker >= p.B * p.Hkv * p.splits) {  // a dense-rest worker, or none
    dense_worker<GQ, BF16>(p, worker - p.B * p.Hkv * p.splits, lane, (float*)lds);
    return;
  }
  const int split = __builtin_amdgcn_readfirstlane(worker % p.splits);
  const int bh = __builtin_amdgcn_readfirstlane(worker / p.splits);
  const int b = __builtin_amdgcn_readfirstlane(bh / p.Hkv), kvh = __builtin_amdgcn_readfirstlane(bh % p.Hkv);
  const int hp0 = __builtin_amdgcn_readfirstlane((int)(((int64_t)split * 2 * p.count) / p.splits));
  const int hp1 = __builtin_amdgcn_readfirstlane((int)(((int64_t)(split + 1) * 2 * p.count) / p.splits));

  // ---- per-lane constants ----
  constexpr int ktpb = 8 / KB, vtpb = 8 / VB;
  const int slot = n >> 2, head = n & 3;                   // slot-layout A row n = 4 * slot + head
  constexpr int kf = key_rows_per_stage(KB);
  const int krow = M.kc + 8 * KB * kf * kq + 4 * (n / ktpb);  // key code dword of channel kq, + 32 KB kf per block
  const int kshift = KB * (n % ktpb);
  const int vdw = 4 * (n / vtpb);                          // value code dword in a row (tile 0)
  const int vshift = VB * (n % vtpb);
  const int vch0 = code_index<VB>(n, 0);                   // first channel of the lane (tile 0)
  const int vg0 = vch0 / p.vg, vg1 = (vch0 + 64) / p.vg;   // value groups of tiles 0 and 1
  int aq[4];  // one row group: P V A sources, the weight row of the lane's head at its slot, else zeros
#pragma unroll
  for (int i = 0; i < 4; ++i) aq[i] = (i == slot && head < GQ) ? M.pt + kPtRow * head + 2 * kq : M.zero + 2 * kq;
  // two row groups: the non-zero A value's LDS address per group (query, weights), placed by slot_a
  const uint2 asel = slot_sel(slot, head < GH);
  int qsrc[RG], wsrc[RG];
#pragma unroll
  for (int g = 0; g < RG; ++g) {
    qsrc[g] = M.q16 + 2 * ((4 * g + head) * kD + kq);
    wsrc[g] = M.pt + kPtRow * (4 * g + head) + 2 * kq;
  }

  // ---- running state ----
  // S[g]: lane (n, kq) holds rows 4g + 0..3 of half-page token code_index<KB>(n, kq).
  // O[g][t]: lane (n, kq) holds rows 4g + 0..3 of channel 64 t + code_index<VB>(n, kq).
  float m_run[RG][4], l_part[RG][4];
  float4v O[RG][2];
#pragma unroll
  for (int g = 0; g < RG; ++g) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      m_run[g][i] = -INFINITY;
      l_part[g][i] = 0.f;
    }
    O[g][0] = O[g][1] = float4v{0.f, 0.f, 0.f, 0.f};
  }

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
  half4 qa[RG == 1 ? kD / 4 : 1];  // one row group: Q K A operands, q[head][4cb + kq] at half `slot`
  if constexpr (RG == 1) {
    const uint16_t* q16 = (const uint16_t*)(lds + M.q16);
#pragma unroll
    for (int cb = 0; cb < kD / 4; ++cb) {
      const _Float16 v = __builtin_bit_cast(_Float16, q16[head * kD + 4 * cb + kq]);
#pragma unroll
      for (int i = 0; i < 4; ++i) qa[cb][i] = i == slot ? v : (_Float16)0.f;
    }
  }
  if (hp0 < hp1) {
    const PageAddr a0 = page_addr(descriptor(p.segs, p.first + (hp0 >> 1)), bh);
    issue_keys_u(M, lds, a0, KB, hp0 & 1, lane);
    issue_values_u(M, lds, a0, VB, gv, hp0 & 1, lane);
  }
  const float c2 = ldexpf(p.scale * kLog2e, qexp);
  const uint32_t kmask = code_mask<KB>(), vmask = code_mask<VB>();
  // table addressing: block cb's key tables at kt + 128 cb (the lane's channel
  // 4 cb + kq at + 32 kq), token group tg's value tables of tile t at
  // vt + 1024 vg_t + 128 (tg mod 8) (the lane's token at + 32 kq); the bases'
  // low bytes are zero, byte j of a selector is 2 code_j + 32 kq
  const uint32_t kq32 = 0x20202020u * (uint32_t)kq;
  const uint32_t krot = (uint32_t)(kshift - 1) & 31u, vrot = (uint32_t)(vshift - 1) & 31u;
  const uint32_t kt_base = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void*)(lds + M.kt));
  const uint32_t vt_base0 = (uint32_t)(uintptr_t)(lds_void*)(lds + M.vt + kQuarterTok * kTable * vg0);
  const uint32_t vt_base1 = (uint32_t)(uintptr_t)(lds_void*)(lds + M.vt + kQuarterTok * kTable * vg1);

#pragma unroll 1
  for (int hq = hp0; hq < hp1; ++hq) {
    const bool has_next = hq + 1 < hp1;
    PageAddr nxt;
    if (has_next) nxt = page_addr(descriptor(p.segs, p.first + ((hq + 1) >> 1)), bh);
    const int nh = (hq + 1) & 1;
    // the next half needs new key rows unless it is the second half of a page staged whole
    const bool keys_next = has_next && (kf == 1 || nh == 0);
    // outstanding, oldest first: key scales + codes (if staged for this half), values (this half)
    vm_wait(n_value_loads_u(VB, gv));
    if (hq == hp0 || kf == 1 || (hq & 1) == 0) {  // keys staged for this half: their (s, s, z, z) table
      if constexpr (KT) build_key_tables<KB, BF16>(M, lds, lane);
      else build_sz_table(lds, M.kt, M.ks, M.kz, kD, lane);
      lds_sync();
    }

    // ---- S = Q K over the half's 64 tokens ----
    float4v S[RG];
#pragma unroll
    for (int g = 0; g < RG; ++g) S[g] = float4v{0.f, 0.f, 0.f, 0.f};
    {
      constexpr int kAhead = KT ? 3 : 2;  // code words read ahead (with tables: gathered two ahead)
      uint32_t w[kD / 4];
      uint2 sz[kD / 4];
      half4 bk[kD / 4];  // with key tables: block cb's B operand, gathered one block ahead
      const int kh = krow + (kf == 2 ? 8 * KB * (hq & 1) : 0);
      auto load_cb = [&](int c) {
        w[c] = lds_u32(lds, kh + 32 * KB * kf * c);
        if constexpr (!KT) sz[c] = *(const uint2*)(lds + M.kt + 8 * (4 * c + kq));
      };
      auto gather_cb = [&](int c) { bk[c] = gather4(kt_base, twice_code_bytes<KB>(w[c], krot, kq32), 4 * kTable * c); };
#pragma unroll
      for (int c = 0; c < kAhead; ++c) load_cb(c);
      if constexpr (KT) {
        gather_cb(0);
        gather_cb(1);
      }
      half4 pend;  // even block's B operand, waiting for the odd one
#pragma unroll
      for (int cb = 0; cb < kD / 4; ++cb) {
        if (cb + kAhead < kD / 4) load_cb(cb + kAhead);
        half4 b;
        if constexpr (KT) {
          if (cb + 2 < kD / 4) gather_cb(cb + 2);
          b = bk[cb];
        } else {
          b = dequant4<KB, BF16>((w[cb] >> kshift) & kmask, sz[cb]);
        }
        if (cb & 1) {  // blocks cb - 1, cb in one K = 32 MFMA
          if constexpr (RG == 1) {
            S[0] = mma2(qa[cb - 1], qa[cb], pend, b, S[0]);
          } else {
#pragma unroll
            for (int g = 0; g < RG; ++g)
              S[g] = mma2(slot_a(*(const uint16_t*)(lds + qsrc[g] + 8 * (cb - 1)), asel),
                          slot_a(*(const uint16_t*)(lds + qsrc[g] + 8 * cb), asel), pend, b, S[g]);
          }
        } else {
          pend = b;
        }
      }
    }
    lds_sync();
    if (keys_next) issue_keys_u(M, lds, nxt, KB, nh, lane);
    // this half's values are older than the next half's key loads issued since
    vm_wait(keys_next ? n_key_loads_u(KB) : 0);
    if constexpr (!VT) build_sz_table(lds, M.vt, M.vs, M.vz, kHalfTok * gv, lane);

    // ---- online softmax in base 2 ----
    {
      float x[RG][4];
      bool over = false;
#pragma unroll
      for (int g = 0; g < RG; ++g) {
#pragma unroll
        for (int i = 0; i < GH; ++i) {
          x[g][i] = S[g][i] * c2;
          over |= x[g][i] > m_run[g][i] + kSlack;
        }
      }
      if (__ballot(over) != 0ull) {
#pragma unroll
        for (int g = 0; g < RG; ++g) {
#pragma unroll
          for (int i = 0; i < GH; ++i) {
            const float m_new = uniform(fmaxf(m_run[g][i], wave_max64(x[g][i])));
            const float alpha = __builtin_amdgcn_exp2f(m_run[g][i] - m_new);
            O[g][0][i] *= alpha;
            O[g][1][i] *= alpha;
            l_part[g][i] *= alpha;
            m_run[g][i] = m_new;
          }
        }
      }
      uint16_t* pt = (uint16_t*)(lds + M.pt);
      const int tok = code_index<KB>(n, kq);
#pragma unroll
      for (int g = 0; g < RG; ++g) {
#pragma unroll
        for (int i = 0; i < GH; ++i) {
          const float pv = __builtin_amdgcn_exp2f(x[g][i] - m_run[g][i]);
          l_part[g][i] += pv;
          pt[(4 * g + i) * (kPtRow / 2) + tok] = __builtin_bit_cast(uint16_t, (_Float16)pv);
        }
      }
    }
    lds_sync();

    // ---- O += P V: token group tg = tokens 4 tg .. 4 tg + 3, lane's token 4 tg + kq ----
    // (with value tables: per quarter page, the quarter's tables first; a
    // group's codes are read three groups ahead, its B operands gathered two
    // ahead, and its A operand formed from the one non-zero weight, slot_a)
    {
      constexpr int kQuarters = VT ? kHalfTok / kQuarterTok : 1;
      constexpr int kGroups = kHalfTok / 4 / kQuarters;  // token groups per table build
      constexpr int kLoadAhead = VT ? 3 : 1;
      half4 a[RG][kHalfTok / 4];
      uint32_t w0[kHalfTok / 4], w1[kHalfTok / 4];
      uint2 sz0[kHalfTok / 4], sz1[kHalfTok / 4];
      half4 bv0[kHalfTok / 4], bv1[kHalfTok / 4];
      auto load_tg = [&](int tg) {
        const int t = 4 * tg + kq;
        if constexpr (RG == 1 && !VT) {
          a[0][tg] = load_a(lds, aq, 8 * tg);
        } else {
#pragma unroll
          for (int g = 0; g < RG; ++g) a[g][tg] = slot_a(*(const uint16_t*)(lds + wsrc[g] + 8 * tg), asel);
        }
        w0[tg] = lds_u32(lds, M.vc + 16 * VB * t + vdw);
        w1[tg] = lds_u32(lds, M.vc + 16 * VB * t + 8 * VB + vdw);
        if constexpr (!VT) {
          sz0[tg] = *(const uint2*)(lds + M.vt + 8 * (t * gv + vg0));
          sz1[tg] = *(const uint2*)(lds + M.vt + 8 * (t * gv + vg1));
        }
      };
      auto gather_tg = [&](int tg) {
        const int off = 4 * kTable * (tg % (kQuarterTok / 4));
        bv0[tg] = gather4(vt_base0, twice_code_bytes<VB>(w0[tg], vrot, kq32), off);
        bv1[tg] = gather4(vt_base1, twice_code_bytes<VB>(w1[tg], vrot, kq32), off);
      };
      half4 p0, p1;  // even group's B operands, waiting for the odd one
#pragma unroll
      for (int qr = 0; qr < kQuarters; ++qr) {
        if constexpr (VT) {
          if (qr > 0) lds_sync();  // the previous quarter's gathers are done
          build_value_tables<VB, BF16>(M, lds, gv, qr, lane);
          lds_sync();
        }
        const int tg0 = kGroups * qr;
#pragma unroll
        for (int i = 0; i < kLoadAhead; ++i) load_tg(tg0 + i);
        if constexpr (VT) {
          gather_tg(tg0);
          gather_tg(tg0 + 1);
        }
#pragma unroll
        for (int i = 0; i < kGroups; ++i) {
          const int tg = tg0 + i;
          if (i + kLoadAhead < kGroups) load_tg(tg + kLoadAhead);
          half4 b0, b1;
          if constexpr (VT) {
            if (i + 2 < kGroups) gather_tg(tg + 2);
            b0 = bv0[tg];
            b1 = bv1[tg];
          } else {
            b0 = dequant4<VB, BF16>((w0[tg] >> vshift) & vmask, sz0[tg]);
            b1 = dequant4<VB, BF16>((w1[tg] >> vshift) & vmask, sz1[tg]);
          }
          if (tg & 1) {  // token groups tg - 1, tg in one K = 32 MFMA per tile
#pragma unroll
            for (int g = 0; g < RG; ++g) {
              O[g][0] = mma2(a[g][tg - 1], a[g][tg], p0, b0, O[g][0]);
              O[g][1] = mma2(a[g][tg - 1], a[g][tg], p1, b1, O[g][1]);
            }
          } else {
            p0 = b0;
            p1 = b1;
          }
        }
      }
    }
    lds_sync();
    if (has_next) issue_values_u(M, lds, nxt, VB, gv, nh, lane);
  }

  // ---- partial state ----
  const int ch = code_index<VB>(n, kq);
#pragma unroll
  for (int g = 0; g < RG; ++g) {
#pragma unroll
    for (int i = 0; i < GH; ++i) {
      const float l = wave_sum64(l_part[g][i]);
      const int hq = kvh * GQ + 4 * g + i;
      float* rec = p.ws + (((int64_t)b * p.Hq + hq) * p.split_stride + split) * (kD + 2);
      if (lane == 0) {
        rec[0] = m_run[g][i] * kLn2;
        rec[1] = l;
      }
      rec[2 + ch] = O[g][0][i];
      rec[2 + 64 + ch] = O[g][1][i];
    }
  }
}

}  // namespace

namespace dkv {

// The kernel waits until at most one half page's key or value loads are in
// flight; vm_wait takes counts below 16.
// Value tables when the values are 2- or 4-bit, there are at most 4 query
// rows and at most two value groups per token.
static bool use_value_tables(int vb, int gq, int gv) { return value_tables_ok(vb, gq) && gv <= 2; }

size_t uniform_decode_wave_lds_bytes(int kb, int vb, int gv) {
  return (size_t)umap(kb, vb, gv, 1, key_tables(kb, 1), use_value_tables(vb, 1, gv)).bytes;
}

int uniform_decode_max_loads(int kb, int vb, int gv) {
  return n_key_loads_u(kb) > n_value_loads_u(vb, gv) ? n_key_loads_u(kb) : n_value_loads_u(vb, gv);
}

template <int G, int K, int V>
static void launch_uniform_kernel(bool vtab, bool bf16, dim3 grid, dim3 block, size_t lds, hipStream_t stream,
                                  const FastParams& p) {
  if constexpr (value_tables_ok(V, G)) {
    if (vtab) {
      if (bf16) hipLaunchKernelGGL((decode_pages_uniform<G, K, V, true, true>), grid, block, lds, stream, p);
      else hipLaunchKernelGGL((decode_pages_uniform<G, K, V, false, true>), grid, block, lds, stream, p);
      return;
    }
  }
  if (bf16) hipLaunchKernelGGL((decode_pages_uniform<G, K, V, true, false>), grid, block, lds, stream, p);
  else hipLaunchKernelGGL((decode_pages_uniform<G, K, V, false, false>), grid, block, lds, stream, p);
}

int launch_uniform_decode(const dkv_decode_args& a, int first, int count, int kb, int vb, int vg, int splits,
                          int split_stride, hipStream_t stream, const FusedRest* fused) {
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
  p.np = 0;
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
  const int64_t workers = (int64_t)p.B * p.Hkv * splits + p.dense_workers;
  const dim3 grid((unsigned)((workers + kWaves - 1) / kWaves)), block(256);
  const bool vtab = use_value_tables(vb, p.GQ, p.gv);
  const size_t lds =
      (size_t)kWaves * umap(kb, vb, p.gv, p.GQ > 4 ? 2 : 1, key_tables(kb, p.GQ), vtab).bytes;
  if ((kb != 2 && kb != 4 && kb != 8) || (vb != 2 && vb != 4 && vb != 8)) {
    set_error("uniform page decode supports 2, 4 and 8-bit codes");
    return DKV_ERR_UNSUPPORTED;
  }
  if (p.GQ != 1 && p.GQ != 2 && p.GQ != 4 && p.GQ != 8) {
    set_error("uniform page decode supports 1, 2, 4 or 8 query rows per KV head");
    return DKV_ERR_UNSUPPORTED;
  }
#define DKV_U_LAUNCH(G, K, V) launch_uniform_kernel<G, K, V>(vtab, p.bf16 != 0, grid, block, lds, stream, p)
#define DKV_U_V(G, K)                                   \
  switch (vb) {                                         \
    case 2: DKV_U_LAUNCH(G, K, 2); break;               \
    case 4: DKV_U_LAUNCH(G, K, 4); break;               \
    default: DKV_U_LAUNCH(G, K, 8); break;              \
  }
#define DKV_U_K(G)                                      \
  switch (kb) {                                         \
    case 2: DKV_U_V(G, 2); break;                       \
    case 4: DKV_U_V(G, 4); break;                       \
    default: DKV_U_V(G, 8); break;                      \
  }
  switch (p.GQ) {
    case 1: DKV_U_K(1); break;
    case 2: DKV_U_K(2); break;
    case 4: DKV_U_K(4); break;
    default: DKV_U_K(8); break;
  }
#undef DKV_U_K
#undef DKV_U_V
#undef DKV_U_LAUNCH
  return dkv_check_launch("dkv_decode_attention(uniform pages)");
}

}  // namespace dkv
