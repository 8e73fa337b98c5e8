// LDS read throughput on gfx950 (a measurement probe, not part of the
// library; built and run on its own:
//   hipcc -O3 --offload-arch=gfx950 lds_throughput.hip -o lds_throughput).
//
// Times conflict-free 16-byte reads (each wave its own 4 KB region) and
// 8-byte gathers at random entries of a 2 KB table (the access pattern of a
// 256-entry lookup table indexed by data), with 8 and 16 waves per CU.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdint.h>
#include <stdlib.h>

#define CK(x) do { hipError_t e = (x); if (e != hipSuccess) { printf("HIP error %s at %d\n", hipGetErrorString(e), __LINE__); exit(1);} } while (0)

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int ITERS = 4096;

// each wave reads 16 B per lane, conflict-free, from its own 4 KB region
__global__ void __launch_bounds__(256) lds_b128(uint32_t* out, int salt) {
  __shared__ __attribute__((aligned(16))) uint8_t s[16384];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int i = threadIdx.x; i < 4096; i += 256) ((uint32_t*)s)[i] = i * 2654435761u + salt;
  __syncthreads();
  const uint8_t* base = s + wave * 4096 + 16 * lane;
  u32x4 acc = {0, 0, 0, 0};
#pragma unroll 8
  for (int it = 0; it < ITERS; ++it) {
    const int off = (it & 3) * 1024;
    u32x4 v = *(const u32x4*)(base + off);
    acc ^= v;
    asm volatile("" : "+v"(acc));
  }
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x12345678u) out[0] = 1;
}

// each lane gathers 8 B from a 2 KB table at 8 * (pseudo-random byte)
__global__ void __launch_bounds__(256) lds_gather_b64(uint32_t* out, int salt) {
  __shared__ __attribute__((aligned(16))) uint8_t s[2048];
  for (int i = threadIdx.x; i < 512; i += 256) ((uint32_t*)s)[i] = i * 2654435761u + salt;
  __syncthreads();
  uint32_t x = (threadIdx.x * 2654435761u) ^ salt;
  u32x2 acc = {0, 0};
#pragma unroll 8
  for (int it = 0; it < ITERS; ++it) {
    x = x * 1664525u + 1013904223u;
    const uint32_t addr = ((x >> 24) & 0xff) * 8;
    u32x2 v = *(const u32x2*)(s + addr);
    acc ^= v;
  }
  if ((acc.x ^ acc.y) == 0x12345678u) out[0] = 1;
}

template <typename F>
static float time_ms(F launch, int reps) {
  hipEvent_t a, b;
  CK(hipEventCreate(&a)); CK(hipEventCreate(&b));
  launch(); launch();
  CK(hipDeviceSynchronize());
  CK(hipEventRecord(a, 0));
  for (int i = 0; i < reps; ++i) launch();
  CK(hipEventRecord(b, 0));
  CK(hipEventSynchronize(b));
  float ms; CK(hipEventElapsedTime(&ms, a, b));
  return ms / reps;
}

int main() {
  uint32_t* out;
  CK(hipMalloc(&out, 64));
  hipDeviceProp_t prop;
  CK(hipGetDeviceProperties(&prop, 0));
  const int cus = prop.multiProcessorCount;
  printf("CUs %d, clock %d kHz\n", cus, prop.clockRate);
  for (int wpc : {8, 16}) {  // waves per CU
    const int blocks = cus * wpc / 4;
    const double waves = (double)blocks * 4;
    float ms = time_ms([&] { lds_b128<<<blocks, 256>>>(out, 1); }, 10);
    double bytes = waves * ITERS * 64 * 16;
    printf("ds_read_b128 conflict-free, %2d waves/CU: %.3f ms, %.1f B/clk/CU at 2.1 GHz (%.2f TB/s chip)\n", wpc, ms,
           bytes / (ms * 1e-3) / cus / 2.1e9, bytes / (ms * 1e-3) / 1e12);
    ms = time_ms([&] { lds_gather_b64<<<blocks, 256>>>(out, 1); }, 10);
    bytes = waves * ITERS * 64 * 8;
    printf("ds_read_b64 random gather 2 KB, %2d waves/CU: %.3f ms, %.1f B/clk/CU, %.2f cycles per wave-instruction per CU\n",
           wpc, ms, bytes / (ms * 1e-3) / cus / 2.1e9, (ms * 1e-3 * 2.1e9) / (waves / cus * ITERS));
    fflush(stdout);
  }
  return 0;
}
