/* Host check of the reciprocal-form division the quantize kernels use:
 * q = RN(a y), r = RN(a - b q) (exact with an fma), q' = RN(q + r y), y = RN(1 / b).
 *
 *   qmax <n>       every positive finite fp32 a, b = n: prints the number of q' != RN(a / b).
 *   pairs bf16|f16 every 16-bit a >= 0, b >= 2^-22 with a <= 260 b, as the
 *                  per-element division diff / scale sees them: prints the number of
 *                  mismatches and the largest RN(a / b) among them.
 * Built with gcc -O2 -fopenmp -ffp-contract=off; fmaf is the C library's fused multiply-add. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t bits_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float recip_div(float a, float b, float y) {
  const float q = a * y;
  const float r = fmaf(-q, b, a);
  return fmaf(r, y, q);
}
static float f16_value(uint32_t h) {
  const uint32_t e = (h >> 10) & 31, m = h & 1023;
  if (e == 0) return ldexpf((float)m, -24);
  return from_bits(((e + 112) << 23) | (m << 13));
}

int main(int argc, char** argv) {
  if (argc == 3 && strcmp(argv[1], "qmax") == 0) {
    const float b = (float)atoi(argv[2]), y = 1.0f / b;
    long long bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static, 1 << 16)
    for (long long u = 1; u < 0x7f800000LL; ++u) {
      const float a = from_bits((uint32_t)u);
      bad += bits_of(recip_div(a, b, y)) != bits_of(a / b);
    }
    printf("%lld\n", bad);
    return 0;
  }
  if (argc == 3 && strcmp(argv[1], "pairs") == 0) {
    const int f16 = strcmp(argv[2], "f16") == 0;
    const uint32_t end = f16 ? 0x7c00u : 0x7f80u;
    long long bad = 0;
    float worst = 0.0f;
#pragma omp parallel for reduction(+ : bad) reduction(max : worst) schedule(dynamic, 64)
    for (uint32_t bb = 1; bb < end; ++bb) {
      const float b = f16 ? f16_value(bb) : from_bits(bb << 16);
      if (b < 0x1p-22f) continue;
      const float y = 1.0f / b;
      for (uint32_t aa = 0; aa < end; ++aa) {
        const float a = f16 ? f16_value(aa) : from_bits(aa << 16);
        if (a > 260.0f * b) break;
        const float ref = a / b;
        if (bits_of(recip_div(a, b, y)) != bits_of(ref)) {
          ++bad;
          worst = fmaxf(worst, ref);
        }
      }
    }
    printf("%lld %a\n", bad, worst);
    return 0;
  }
  fprintf(stderr, "usage: div_check qmax <n> | pairs bf16|f16\n");
  return 2;
}
