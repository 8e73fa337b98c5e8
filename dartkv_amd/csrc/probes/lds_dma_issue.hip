// Probe (not part of the library): what issuing LDS DMA (global_load_lds_dwordx4)
// costs the issuing wave on gfx950, and which counter tracks its completion.
//
// Each wave issues N back-to-back 1 KiB copies from a cold 16 KiB chunk of its
// own into its LDS region, then reads the shader clock (the issue time), waits
// for vmcnt(0) and reads it again (the completion time).  A second kernel
// waits on lgkmcnt(0) first and then on vmcnt(0): if LDS DMA were tracked by
// lgkmcnt, the second wait would find nothing left to wait for.
//
//   hipcc -O3 --offload-arch=gfx950 lds_dma_issue.hip -o /tmp/lds_dma_issue && /tmp/lds_dma_issue
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#define CHECK(x)                                                             \
  do {                                                                       \
    hipError_t e_ = (x);                                                     \
    if (e_ != hipSuccess) {                                                  \
      fprintf(stderr, "%s failed: %s\n", #x, hipGetErrorString(e_));         \
      return 1;                                                              \
    }                                                                        \
  } while (0)

constexpr int kChunk = 16384;  // bytes of source per wave, and LDS per wave

__device__ __forceinline__ void dma16(const uint8_t* src, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds_addr) : "memory");
}

template <int N>
__global__ void issue_then_wait(const uint8_t* buf, unsigned long long* out) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int gw = blockIdx.x * (blockDim.x >> 6) + wave;
  const uint8_t* src = buf + (size_t)gw * kChunk;
  const uint32_t base =
      __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)(smem + wave * kChunk));
  const unsigned long long t0 = __builtin_readcyclecounter();
#pragma unroll
  for (int i = 0; i < N; ++i) dma16(src + 1024 * i + 16 * lane, base + 1024 * i);
  const unsigned long long t1 = __builtin_readcyclecounter();
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  const unsigned long long t2 = __builtin_readcyclecounter();
  if (lane == 0) {
    out[2 * gw] = t1 - t0;
    out[2 * gw + 1] = t2 - t1;
  }
}

// lgkmcnt(0) first, then vmcnt(0): the time each wait takes.
__global__ void lgkm_then_vm(const uint8_t* buf, unsigned long long* out) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const uint8_t* src = buf + (size_t)blockIdx.x * kChunk;
  const uint32_t base = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)smem);
#pragma unroll
  for (int i = 0; i < 8; ++i) dma16(src + 1024 * i + 16 * lane, base + 1024 * i);
  const unsigned long long t0 = __builtin_readcyclecounter();
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  const unsigned long long t1 = __builtin_readcyclecounter();
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  const unsigned long long t2 = __builtin_readcyclecounter();
  if (lane == 0) {
    out[2 * blockIdx.x] = t1 - t0;
    out[2 * blockIdx.x + 1] = t2 - t1;
  }
}

static int report(const char* what, unsigned long long* dev, int n) {
  unsigned long long* h = new unsigned long long[2 * n];
  CHECK(hipMemcpy(h, dev, 16 * (size_t)n, hipMemcpyDeviceToHost));
  double a = 0, b = 0, amax = 0;
  for (int i = 0; i < n; ++i) {
    a += h[2 * i];
    b += h[2 * i + 1];
    if (h[2 * i] > amax) amax = h[2 * i];
  }
  printf("%s: %.0f (max %.0f) then %.0f cycles\n", what, a / n, amax, b / n);
  delete[] h;
  return 0;
}

template <int N>
static int run(const uint8_t* buf, unsigned long long* out, uint8_t* flush, int blocks, int waves) {
  CHECK(hipMemset(flush, 3, 1ull << 30));  // evicts the source from L2 and the Infinity Cache
  hipLaunchKernelGGL(issue_then_wait<N>, dim3(blocks), dim3(64 * waves), kChunk * waves, 0, buf, out);
  CHECK(hipGetLastError());
  CHECK(hipDeviceSynchronize());
  char what[128];
  snprintf(what, sizeof what, "N=%2d copies, %4d workgroups of %d waves: issue cycles", N, blocks, waves);
  return report(what, out, blocks * waves);
}

int main() {
  const int max_waves = 1024 * 8;
  uint8_t *buf, *flush;
  unsigned long long* out;
  CHECK(hipMalloc(&buf, (size_t)max_waves * kChunk));
  CHECK(hipMemset(buf, 1, (size_t)max_waves * kChunk));
  CHECK(hipMalloc(&out, 16 * (size_t)max_waves));
  CHECK(hipMalloc(&flush, 1ull << 30));
  int rc = 0;
  for (int waves : {1, 8}) {
    for (int blocks : {256, 1024}) {
      rc |= run<4>(buf, out, flush, blocks, waves);
      rc |= run<8>(buf, out, flush, blocks, waves);
      rc |= run<16>(buf, out, flush, blocks, waves);
    }
  }
  CHECK(hipMemset(flush, 3, 1ull << 30));
  hipLaunchKernelGGL(lgkm_then_vm, dim3(256), dim3(64), kChunk, 0, buf, out);
  CHECK(hipGetLastError());
  CHECK(hipDeviceSynchronize());
  rc |= report("8 copies, then s_waitcnt lgkmcnt(0) / vmcnt(0)", out, 256);
  CHECK(hipFree(buf));
  CHECK(hipFree(out));
  CHECK(hipFree(flush));
  return rc;
}
