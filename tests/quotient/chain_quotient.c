/*
 * Exhaustive host check of the quantizers' quotient step for 16-bit sources.
 *
 * The reference's chain (quantization.py:167-168, mixed.py:205-215) computes, in the source dtype,
 * q = round_src(d / s) with d = round_src(x - min) and s the group scale, and keeps rint(q) (then the
 * clamp).  In the source dtype a division is an fp32 IEEE division rounded to the source dtype.  The HIP
 * kernels compute the fp32 quotient as one product d * y with y = RN(1 / s) instead.  For every 16-bit
 * d >= 0 and s >= SMIN (the smallest scale the eps clamp of the group range allows) with d / s < 256,
 * this program checks that rint(round_src(RN(d * y))) == rint(round_src(RN(d / s))), and, as a control,
 * that the product alone is not always equal to the quotient before rounding (the check would be vacuous
 * otherwise).  Prints "ok <dtype> <pairs> <differing products>" per dtype and exits 0, or the first
 * counterexamples.
 * Built by tests/test_chain_quotient.py with clang (for _Float16) and -ffp-contract=off.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#define SMIN 3.8e-7f
#define NTHREADS 8

static float from_bits(uint32_t v) { float x; memcpy(&x, &v, 4); return x; }
static uint32_t to_bits(float x) { uint32_t v; memcpy(&v, &x, 4); return v; }
static float round_bf16(float x) {  /* nearest even, finite inputs */
  const uint32_t v = to_bits(x);
  return from_bits((v + 0x7fffu + ((v >> 16) & 1u)) & 0xffff0000u);
}
static float round_f16(float x) { return (float)(_Float16)x; }
static float bf16_value(uint32_t i) { return from_bits(i << 16); }
static float f16_value(uint32_t i) { uint16_t b = (uint16_t)i; _Float16 h; memcpy(&h, &b, 2); return (float)h; }

struct job { int fp16; uint32_t s_lo, s_hi; long long pairs, code_bad, raw_diff; };

static void* run(void* p) {
  struct job* j = (struct job*)p;
  const uint32_t n = j->fp16 ? 0x7c00u : 0x7f80u;  /* positive finite encodings */
  for (uint32_t si = j->s_lo; si < j->s_hi; ++si) {
    const float s = j->fp16 ? f16_value(si) : bf16_value(si);
    if (!(s >= SMIN)) continue;
    const float y = 1.0f / s;
    for (uint32_t di = 0; di < n; ++di) {
      const float d = j->fp16 ? f16_value(di) : bf16_value(di);
      if (d >= 256.0f * s) break;
      const float exact = d / s, prod = d * y;
      const float qe = j->fp16 ? round_f16(exact) : round_bf16(exact);
      const float qp = j->fp16 ? round_f16(prod) : round_bf16(prod);
      j->pairs++;
      if (exact != prod) j->raw_diff++;
      if (rintf(qe) != rintf(qp)) {
        if (j->code_bad++ < 4) printf("%s s=%a d=%a exact=%a product=%a\n", j->fp16 ? "f16" : "bf16", s, d, qe, qp);
      }
    }
  }
  return NULL;
}

int main(void) {
  int failed = 0;
  for (int fp16 = 0; fp16 < 2; ++fp16) {
    const uint32_t n = fp16 ? 0x7c00u : 0x7f80u;
    pthread_t th[NTHREADS];
    struct job jobs[NTHREADS];
    for (int t = 0; t < NTHREADS; ++t) {
      jobs[t] = (struct job){fp16, 1 + (n - 1) * (uint32_t)t / NTHREADS, 1 + (n - 1) * (uint32_t)(t + 1) / NTHREADS, 0, 0, 0};
      pthread_create(&th[t], NULL, run, &jobs[t]);
    }
    long long pairs = 0, bad = 0, diff = 0;
    for (int t = 0; t < NTHREADS; ++t) {
      pthread_join(th[t], NULL);
      pairs += jobs[t].pairs;
      bad += jobs[t].code_bad;
      diff += jobs[t].raw_diff;
    }
    printf("%s %s %lld %lld\n", bad == 0 && diff > 0 ? "ok" : "FAIL", fp16 ? "f16" : "bf16", pairs, diff);
    failed |= bad != 0 || diff == 0;
  }
  return failed;
}
