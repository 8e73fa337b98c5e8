// Dense token-row copies of an append in one launch: the cache's sink tokens
// and its held tail are kept in the source dtype (reference
// src/dart/cache.py:183-185 clones the sink tokens, :417-418 and :451-467 the
// pending tail), and an append that quantizes pages makes up to four such
// copies after its quantize launches.  As separate torch copies they ran one
// small kernel each, back to back on the stream; here every block's rows are
// one index space of units (dkv_copy.h), one unit per thread.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dkv_capi_util.h"
#include "dkv_copy.h"

namespace {

constexpr int kCopyThreads = 256;

__global__ void __launch_bounds__(kCopyThreads) copy_token_blocks(dkv::CopyParams p) {
  const int64_t u = (int64_t)blockIdx.x * kCopyThreads + threadIdx.x;
  if (u < p.first[p.n]) dkv::copy_token_unit(p, u);
}

}  // namespace

extern "C" int dkv_copy_token_blocks(const dkv_copy_block* blocks, int64_t n_blocks, void* stream) {
  dkv::CopyParams p;
  const int rc = dkv::prepare_copies(blocks, n_blocks, p, "dkv_copy_token_blocks");
  if (rc != DKV_OK) return rc;
  const int64_t units = p.first[p.n];
  if (units == 0) return DKV_OK;
  const int64_t grid = (units + kCopyThreads - 1) / kCopyThreads;
  hipLaunchKernelGGL(copy_token_blocks, dim3((unsigned)grid), dim3(kCopyThreads), 0, (hipStream_t)stream, p);
  return dkv_check_launch("dkv_copy_token_blocks");
}
