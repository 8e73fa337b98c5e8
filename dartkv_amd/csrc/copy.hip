// Dense token-row copies of an append in one launch: the cache's sink tokens
// and its held tail are kept in the source dtype (reference
// src/dart/cache.py:183-185 clones the sink tokens, :417-418 and :451-467 the
// pending tail), and an append that quantizes pages makes up to four such
// copies after its quantize launches.  As separate torch copies they ran one
// small kernel each, back to back on the stream; here every block's rows are
// one index space of 16-byte (or narrower, when the addresses and strides do
// not allow 16) units, one unit per thread.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dkv_capi_util.h"

namespace {

constexpr int kCopyThreads = 256;

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

__global__ void __launch_bounds__(kCopyThreads) copy_token_blocks(CopyParams p) {
  const int64_t u = (int64_t)blockIdx.x * kCopyThreads + threadIdx.x;
  if (u >= p.first[p.n]) return;
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
int unit_shift(const dkv_copy_block& c) {
  const uint64_t all = (uint64_t)(uintptr_t)c.src | (uint64_t)(uintptr_t)c.dst | (uint64_t)c.row_bytes |
                       (uint64_t)c.src_sb | (uint64_t)c.src_sh | (uint64_t)c.src_st | (uint64_t)c.dst_sb |
                       (uint64_t)c.dst_sh | (uint64_t)c.dst_st;
  int s = 0;
  while (s < 4 && !(all & ((2ull << s) - 1))) ++s;
  return s;
}

}  // namespace

extern "C" int dkv_copy_token_blocks(const dkv_copy_block* blocks, int64_t n_blocks, void* stream) {
  DKV_CHECK(n_blocks >= 0 && n_blocks <= DKV_COPY_MAX_BLOCKS, DKV_ERR_INVALID,
            "dkv_copy_token_blocks: n_blocks must be in [0, %d]", DKV_COPY_MAX_BLOCKS);
  DKV_CHECK(n_blocks == 0 || blocks != nullptr, DKV_ERR_INVALID, "dkv_copy_token_blocks: blocks is NULL");
  CopyParams p{};
  int64_t units = 0;
  for (int64_t i = 0; i < n_blocks; ++i) {
    const dkv_copy_block& c = blocks[i];
    DKV_CHECK(c.B >= 0 && c.H >= 0 && c.T >= 0 && c.row_bytes >= 0, DKV_ERR_INVALID,
              "dkv_copy_token_blocks: block %lld has a negative size", (long long)i);
    if (c.B == 0 || c.H == 0 || c.T == 0 || c.row_bytes == 0) continue;
    DKV_CHECK(c.src != nullptr && c.dst != nullptr, DKV_ERR_INVALID, "dkv_copy_token_blocks: block %lld: NULL pointer",
              (long long)i);
    const int s = unit_shift(c);
    p.blk[p.n] = c;
    p.unit_shift[p.n] = s;
    p.first[p.n] = units;
    units += c.B * c.H * c.T * (c.row_bytes >> s);
    ++p.n;
  }
  p.first[p.n] = units;
  if (units == 0) return DKV_OK;
  const int64_t grid = (units + kCopyThreads - 1) / kCopyThreads;
  DKV_CHECK(grid <= 0x7fffffff, DKV_ERR_UNSUPPORTED, "dkv_copy_token_blocks: too many rows for one launch");
  hipLaunchKernelGGL(copy_token_blocks, dim3((unsigned)grid), dim3(kCopyThreads), 0, (hipStream_t)stream, p);
  return dkv_check_launch("dkv_copy_token_blocks");
}
