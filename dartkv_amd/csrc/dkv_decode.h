// Internal interface between the decode entry point and the fast page kernel.
#pragma once
#include <hip/hip_runtime.h>

#include "../../include/dartkv.h"

namespace dkv {

struct DecodeParams;

// A page kernel launch that also runs the dense rest (the non-page segments
// and the tail, `chunks` 32-token chunks each), described as the dense
// kernels take it.
struct FusedRest {
  const DecodeParams* rest;
  int chunks;
};

// Loads in flight between a page's value codes and its PV (must be < 16).
int fast_decode_max_loads(int np, int gv);

// LDS bytes one fast-kernel workgroup needs, and one of its waves.
size_t fast_decode_lds_bytes(int np, int gv, int gq);

// Launch the fast kernel over descriptor entries [first, first + count) of
// a.segments (all full 128-token pages with the fast layout), writing splits
// [0, splits) of a workspace whose records hold `split_stride` splits.
int launch_fast_decode(const dkv_decode_args& a, int first, int count, int np, int vg, int splits,
                       int split_stride, hipStream_t stream, const FusedRest* fused = nullptr);

// Uniform pages (KB-bit keys along tokens, VB-bit values along channels):
// the largest load count one wait must cover, and the launch (splits over
// half pages).
int uniform_decode_max_loads(int kb, int vb, int gv);
int launch_uniform_decode(const dkv_decode_args& a, int first, int count, int kb, int vb, int vg, int splits,
                          int split_stride, hipStream_t stream, const FusedRest* fused = nullptr);
// LDS bytes of one wave of the uniform page kernel.
size_t uniform_decode_wave_lds_bytes(int kb, int vb, int gv);

}  // namespace dkv
