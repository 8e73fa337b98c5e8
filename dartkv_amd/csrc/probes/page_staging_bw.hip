// HBM read ceilings for the decode page kernel's staging (a measurement
// probe, not part of the library; built and run on its own:
//   hipcc -O3 --offload-arch=gfx950 page_staging_bw.hip -o page_staging_bw).
//
// On a 1.42 GB buffer (the packed pages of one C5 layer: 512 (batch, kv head)
// blocks x 255 pages x 10,880 bytes) it times
//   * a plain read (grid-stride 16-byte loads into registers);
//   * one contiguous 176 KB chunk per wave, 4 or 8 KB of loads in flight;
//   * the same chunks through LDS with global_load_lds_dwordx4 (the page
//     kernel's copy instruction), a ring of 8 / 16 / 32 KB per wave;
//   * the page kernel's staging alone: per wave a split of one (batch, kv
//     head)'s pages, each page's eight fields (key low codes 4,096 B, value
//     codes 4,096, key high codes 1,024, indices 128, key scale / zero 256
//     each, value scale / zero 512 each) copied to LDS as the kernel does
//     (fourteen copy instructions), one or two pages in flight, for the pool
//     layout the library uses (key fields page-major, value fields
//     token-major) and for an all-(batch, head)-major one, with 18.9 / 12.8 /
//     24.1 KB of LDS per wave (two waves per SIMD or more) and 8 / 16 / 32
//     splits.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <vector>

#define CK(x) do { hipError_t e = (x); if (e != hipSuccess) { printf("HIP error %s at %d\n", hipGetErrorString(e), __LINE__); exit(1);} } while (0)

typedef __attribute__((address_space(3))) void lds_void;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void dma16(const uint8_t* src, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds_addr) : "memory");
}
__device__ __forceinline__ void copy_to_lds(uint8_t* dst, const uint8_t* src, int bytes, int lane) {
  const uint32_t base = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void*)dst);
  for (int off = 0; off < bytes; off += 1024) {
    if (off + 16 * lane < bytes) dma16(src + off + 16 * lane, base + off);
  }
}
__device__ __forceinline__ void wait_all() {
  __builtin_amdgcn_s_waitcnt(0x0070);
  __builtin_amdgcn_wave_barrier();
}

// ---- plain read: grid-stride dwordx4 loads into registers ----
__global__ void __launch_bounds__(256) read_plain(const u32x4* __restrict__ p, size_t n, uint32_t* out) {
  uint32_t acc = 0;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i + 3 * stride < n; i += 4 * stride) {
    u32x4 a = __builtin_nontemporal_load(p + i);
    u32x4 b = __builtin_nontemporal_load(p + i + stride);
    u32x4 c = __builtin_nontemporal_load(p + i + 2 * stride);
    u32x4 d = __builtin_nontemporal_load(p + i + 3 * stride);
    acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
  }
  for (; i < n; i += stride) { u32x4 a = p[i]; acc ^= a.x ^ a.y ^ a.z ^ a.w; }
  if (acc == 0x12345678u) out[0] = acc;
}

// ---- per-wave contiguous chunk, regular loads, U loads (1 KB per wave each) in flight ----
template <int U>
__global__ void __launch_bounds__(256) read_chunks(const uint8_t* __restrict__ p, size_t per_wave, uint32_t* out) {
  const int lane = threadIdx.x & 63;
  const size_t w = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const uint8_t* base = p + w * per_wave;
  uint32_t acc = 0;
  for (size_t off = 0; off < per_wave; off += 1024 * U) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load((const u32x4*)(base + off + 1024 * u + 16 * lane));
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == 0x12345678u) out[0] = acc;
}

// ---- per-wave contiguous chunk through LDS DMA; ring of R KB per wave ----
__global__ void __launch_bounds__(256) read_dma(const uint8_t* __restrict__ p, size_t per_wave, int ring_kb, uint32_t* out) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const size_t w = (size_t)blockIdx.x * 4 + wave;
  uint8_t* lds = smem + wave * ring_kb * 1024;
  const uint8_t* base = p + w * per_wave;
  // issue ring_kb/2 KB, then wait for the older half while the next half is in flight
  const int half = ring_kb / 2;
  int slot = 0;
  for (size_t off = 0; off < per_wave; off += 1024 * half) {
    for (int u = 0; u < half; ++u) copy_to_lds(lds + (slot * half + u) * 1024, base + off + 1024 * u, 1024, lane);
    slot ^= 1;
    // wait until at most `half` loads are outstanding
    if (half >= 15) __builtin_amdgcn_s_waitcnt(0x0070 | 15);
    else if (half == 8) __builtin_amdgcn_s_waitcnt(0x0070 | 8);
    else __builtin_amdgcn_s_waitcnt(0x0070 | 4);
  }
  wait_all();
  uint32_t v = *(uint32_t*)(lds + 4 * lane);
  if (v == 0x12345678u) out[0] = v;
}

// ---- page skeleton: the page kernel's copies without its compute ----
struct Pool {
  const uint8_t *kl, *kh, *ki, *ks, *kz, *vc, *vs, *vz;
  int bh, slots;     // (batch, head) blocks; pages per (batch, head)
  int layout;        // 0: keys page-major [slot][bh], values token-major [bh][rows]; 1: everything [bh][slot]
};

__device__ __forceinline__ void page_ptrs(const Pool& P, int bh, int pg, const uint8_t* q[8]) {
  const int64_t kidx = P.layout == 0 ? (int64_t)pg * P.bh + bh : (int64_t)bh * P.slots + pg;
  const int64_t vidx = (int64_t)bh * P.slots + pg;  // values are [bh][rows] in both
  q[0] = P.kl + kidx * 4096;
  q[1] = P.kh + kidx * 1024;
  q[2] = P.ki + kidx * 128;
  q[3] = P.ks + kidx * 256;
  q[4] = P.kz + kidx * 256;
  q[5] = P.vc + vidx * 4096;
  q[6] = P.vs + vidx * 512;
  q[7] = P.vz + vidx * 512;
}
__device__ __forceinline__ void issue_page(uint8_t* lds, const uint8_t* q[8], int lane) {
  copy_to_lds(lds + 0, q[0], 4096, lane);
  copy_to_lds(lds + 4096, q[5], 4096, lane);
  copy_to_lds(lds + 8192, q[1], 1024, lane);
  copy_to_lds(lds + 9216, q[2], 128, lane);
  copy_to_lds(lds + 9344, q[3], 256, lane);
  copy_to_lds(lds + 9600, q[4], 256, lane);
  copy_to_lds(lds + 9856, q[6], 512, lane);
  copy_to_lds(lds + 10368, q[7], 512, lane);
}

// DEPTH pages in flight per wave (each its own 10,880-byte region); region = bytes of LDS per wave
template <int DEPTH>
__global__ void __launch_bounds__(256) page_skeleton(Pool P, int splits, int region, uint32_t* out) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int worker = blockIdx.x * 4 + wave;
  if (worker >= P.bh * splits) return;
  const int split = worker % splits, bh = worker / splits;
  const int p0 = (int)((int64_t)split * P.slots / splits), p1 = (int)((int64_t)(split + 1) * P.slots / splits);
  uint8_t* lds = smem + wave * region;
  uint32_t acc = 0;
  const uint8_t* q[8];
  for (int d = 0; d < DEPTH && p0 + d < p1; ++d) {
    page_ptrs(P, bh, p0 + d, q);
    issue_page(lds + d * 10880, q, lane);
  }
  for (int pg = p0; pg < p1; ++pg) {
    // oldest page: wait until only the younger pages' 14 loads each are outstanding
    const int younger = (p1 - pg - 1) < (DEPTH - 1) ? (p1 - pg - 1) : (DEPTH - 1);
    if (younger == 0) __builtin_amdgcn_s_waitcnt(0x0070);
    else if (younger == 1) __builtin_amdgcn_s_waitcnt(0x0070 | 14);
    else __builtin_amdgcn_s_waitcnt(0x0070 | 15);  // (DEPTH 3: conservative, vmcnt has 6 bits on gfx9 but keep < 16)
    __builtin_amdgcn_wave_barrier();
    const int r = (pg - p0) % DEPTH;
    acc ^= *(const uint32_t*)(lds + r * 10880 + 4 * lane);
    __builtin_amdgcn_wave_barrier();
    if (pg + DEPTH < p1) {
      page_ptrs(P, bh, pg + DEPTH, q);
      issue_page(lds + r * 10880, q, lane);
    }
  }
  if (acc == 0x12345678u) out[0] = acc;
}

static float time_ms(void (*launch)(void*), void* ctx, int reps) {
  hipEvent_t a, b;
  CK(hipEventCreate(&a)); CK(hipEventCreate(&b));
  launch(ctx); launch(ctx);
  CK(hipDeviceSynchronize());
  CK(hipEventRecord(a, 0));
  for (int i = 0; i < reps; ++i) launch(ctx);
  CK(hipEventRecord(b, 0));
  CK(hipEventSynchronize(b));
  float ms; CK(hipEventElapsedTime(&ms, a, b));
  return ms / reps;
}

struct Ctx {
  const void* buf; size_t bytes; uint32_t* out; Pool P; int splits; int region; int depth; int ring; int kind;
};

static void launch_any(void* v) {
  Ctx& c = *(Ctx*)v;
  switch (c.kind) {
    case 0: read_plain<<<8192, 256>>>((const u32x4*)c.buf, c.bytes / 16, c.out); break;
    case 1: read_chunks<4><<<(unsigned)(c.bytes / (176 * 1024) / 4), 256>>>((const uint8_t*)c.buf, 176 * 1024, c.out); break;
    case 2: read_chunks<8><<<(unsigned)(c.bytes / (176 * 1024) / 4), 256>>>((const uint8_t*)c.buf, 176 * 1024, c.out); break;
    case 3: read_dma<<<(unsigned)(c.bytes / (176 * 1024) / 4), 256, 4 * c.ring * 1024>>>((const uint8_t*)c.buf, 176 * 1024, c.ring, c.out); break;
    case 4: {
      const int workers = c.P.bh * c.splits;
      const unsigned blocks = (workers + 3) / 4;
      if (c.depth == 1) page_skeleton<1><<<blocks, 256, 4 * c.region>>>(c.P, c.splits, c.region, c.out);
      else page_skeleton<2><<<blocks, 256, 4 * c.region>>>(c.P, c.splits, c.region, c.out);
      break;
    }
  }
}

int main(int argc, char** argv) {
  const int BH = 512, SLOTS = 255;
  const size_t page = 10880;
  const size_t total = (size_t)BH * SLOTS * page;  // 1,420,492,800
  // one big allocation carved into fields, sized for the larger of the layouts
  const size_t fsz[8] = {4096, 1024, 128, 256, 256, 4096, 512, 512};
  uint8_t* base;
  CK(hipMalloc(&base, total + 8 * 4096));
  CK(hipMemset(base, 1, total + 8 * 4096));
  uint32_t* out;
  CK(hipMalloc(&out, 64));
  Pool P;
  const uint8_t* f[8];
  size_t off = 0;
  for (int i = 0; i < 8; ++i) { f[i] = base + off; off += (size_t)BH * SLOTS * fsz[i]; off = (off + 4095) / 4096 * 4096; }
  P.kl = f[0]; P.kh = f[1]; P.ki = f[2]; P.ks = f[3]; P.kz = f[4]; P.vc = f[5]; P.vs = f[6]; P.vz = f[7];
  P.bh = BH; P.slots = SLOTS; P.layout = 0;
  Ctx c{base, total, out, P, 16, 18944, 1, 8, 0};
  const int reps = 20;
  auto report = [&](const char* name, float ms) {
    printf("%-48s %8.1f us  %7.1f GB/s  %5.1f %%\n", name, ms * 1e3, total / (ms * 1e-3) / 1e9, total / (ms * 1e-3) / 8e12 * 100);
    fflush(stdout);
  };
  c.kind = 0; report("plain grid-stride dwordx4 (nt)", time_ms(launch_any, &c, reps));
  c.kind = 1; report("per-wave chunk, 4 KB in flight per wave", time_ms(launch_any, &c, reps));
  c.kind = 2; report("per-wave chunk, 8 KB in flight per wave", time_ms(launch_any, &c, reps));
  for (int ring : {8, 16, 32}) {
    c.kind = 3; c.ring = ring;
    char name[96]; snprintf(name, sizeof name, "per-wave chunk via LDS DMA, ring %d KB", ring);
    report(name, time_ms(launch_any, &c, reps));
  }
  c.kind = 4;
  for (int layout : {0, 1}) {
    c.P.layout = layout;
    for (int depth : {1, 2}) {
      for (int region : {18944, 12800, 24064}) {
        if (depth == 2 && region < 2 * 10880) continue;
        for (int splits : {16, 8, 32}) {
          c.depth = depth; c.region = region; c.splits = splits;
          char name[128];
          snprintf(name, sizeof name, "skeleton layout %d depth %d lds/wave %d splits %d", layout, depth, region, splits);
          report(name, time_ms(launch_any, &c, reps));
        }
      }
    }
  }
  CK(hipFree(base));
  CK(hipFree(out));
  return 0;
}
