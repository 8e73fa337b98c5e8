// Dense token-row copies (dkv_copy_block) as one index space of units: every
// block's rows are cut into 16-byte units (or narrower, when the addresses and
// strides do not allow 16), numbered block after block.  Shared by the copy
// launch and by the quantize launches that take an append's copies along.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dkv_capi_util.h"

namespace dkv {

struct CopyParams {
  dkv_copy_block blk[DKV_COPY_MAX_BLOCKS];
  int64_t first[DKV_COPY_MAX_BLOCKS + 1];  // first unit of each block; first[n] = all units
  int unit_shift[DKV_COPY_MAX_BLOCKS];     // log2 of the block's unit size in bytes
  int n;
};

template <typename U>
__device__ __forceinline__ void copy_unit(const char* s, char* d) {
  *(U*)d = *(const U*)s;
}

// Copy unit u (u < p.first[p.n]).
__device__ __forceinline__ void copy_token_unit(const CopyParams& p, int64_t u) {
  int j = 0;
  while (j + 1 < p.n && u >= p.first[j + 1]) ++j;
  const dkv_copy_block& c = p.blk[j];
  const int us = p.unit_shift[j];
  const int64_t per_row = c.row_bytes >> us;
  const int64_t v = u - p.first[j];
  const int64_t row = v / per_row;
  const int64_t off = (v - row * per_row) << us;
  const int64_t t = row % c.T, bh = row / c.T;
  const int64_t h = bh % c.H, b = bh / c.H;
  const char* s = (const char*)c.src + b * c.src_sb + h * c.src_sh + t * c.src_st + off;
  char* d = (char*)c.dst + b * c.dst_sb + h * c.dst_sh + t * c.dst_st + off;
  switch (us) {
    case 4: copy_unit<uint4>(s, d); break;
    case 3: copy_unit<uint2>(s, d); break;
    case 2: copy_unit<uint32_t>(s, d); break;
    case 1: copy_unit<uint16_t>(s, d); break;
    default: copy_unit<uint8_t>(s, d); break;
  }
}

// Largest power of two, at most 16, dividing every address and stride of the
// block and its row length.
inline int copy_unit_shift(const dkv_copy_block& c) {
  const uint64_t all = (uint64_t)(uintptr_t)c.src | (uint64_t)(uintptr_t)c.dst | (uint64_t)c.row_bytes |
                       (uint64_t)c.src_sb | (uint64_t)c.src_sh | (uint64_t)c.src_st | (uint64_t)c.dst_sb |
                       (uint64_t)c.dst_sh | (uint64_t)c.dst_st;
  int s = 0;
  while (s < 4 && !(all & ((2ull << s) - 1))) ++s;
  return s;
}

// Validate `n_blocks` copy blocks and number their units (nothing is launched).
inline int prepare_copies(const dkv_copy_block* blocks, int64_t n_blocks, CopyParams& p, const char* where) {
  DKV_CHECK(n_blocks >= 0 && n_blocks <= DKV_COPY_MAX_BLOCKS, DKV_ERR_INVALID, "%s: n_blocks must be in [0, %d]",
            where, DKV_COPY_MAX_BLOCKS);
  DKV_CHECK(n_blocks == 0 || blocks != nullptr, DKV_ERR_INVALID, "%s: blocks is NULL", where);
  p = CopyParams{};
  int64_t units = 0;
  for (int64_t i = 0; i < n_blocks; ++i) {
    const dkv_copy_block& c = blocks[i];
    DKV_CHECK(c.B >= 0 && c.H >= 0 && c.T >= 0 && c.row_bytes >= 0, DKV_ERR_INVALID,
              "%s: block %lld has a negative size", where, (long long)i);
    if (c.B == 0 || c.H == 0 || c.T == 0 || c.row_bytes == 0) continue;
    DKV_CHECK(c.src != nullptr && c.dst != nullptr, DKV_ERR_INVALID, "%s: block %lld: NULL pointer", where,
              (long long)i);
    const int s = copy_unit_shift(c);
    p.blk[p.n] = c;
    p.unit_shift[p.n] = s;
    p.first[p.n] = units;
    units += c.B * c.H * c.T * (c.row_bytes >> s);
    ++p.n;
  }
  p.first[p.n] = units;
  DKV_CHECK(units / 256 < 0x7fffffffLL, DKV_ERR_UNSUPPORTED, "%s: too many rows for one launch", where);
  return DKV_OK;
}

}  // namespace dkv
