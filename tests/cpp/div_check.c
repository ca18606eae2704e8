/*
 * div_check.c -- CPU check of the temperature division the sampler's kernels
 * use on slices whose logits all lie in the covered range (zdiv with fast =
 * true in mlxforge_amd/csrc/sampler_impl.hpp): Markstein's FMA-corrected
 * quotient
 *     y = RN(1/T), q0 = RN(z*y), r = fma(-q0, T, z), q1 = fma(r, y, q0)
 * (q0 where r is NaN, i.e. for infinite z), against the correctly rounded z / T
 * that src/sample/sampler.cpp:158 computes.
 *
 * Covered range: 2^-24 <= T <= 2^24, and z = 0, +-inf or 2^-96 <= |z| < 2^100.
 * Cases:
 *   bf16  every bf16 z in range x every bf16 T in range        (exhaustive)
 *   f16   every f16 z x every STRIDE-th f16 T in range
 *   f32   N random z (uniform exponent over the range, random mantissa) x
 *         random T, plus z at the two range edges.
 * Prints "cases <n> mismatches <m>" and exits 1 on any mismatch.
 * Build: gcc -O2 -ffp-contract=off div_check.c -lm -lpthread
 * (-DPLANT_NO_CORRECTION drops the correction step, which the check must catch).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define NTHREADS 8

static float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

static float h2f(uint16_t h) {
  const uint32_t s = ((uint32_t)h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 0x1f) return u2f(s | 0x7f800000u | (m << 13));
  if (e == 0) {
    const float v = (float)m * 0x1p-24f;
    return s ? -v : v;
  }
  return u2f(s | ((e - 15 + 127) << 23) | (m << 13));
}

static int z_in_range(float z) {
  const uint32_t az = f2u(z) & 0x7fffffffu;
  if (az == 0 || az == 0x7f800000u) return 1;
  return az >= 0x0f800000u && az < 0x71800000u;
}

static int t_in_range(float t) { return t >= 0x1p-24f && t <= 0x1p24f; }

static float fast_div(float z, float t, float y) {
  const float q0 = z * y;
  const float r = fmaf(-q0, t, z);
  const float q1 = fmaf(r, y, q0);
#ifdef PLANT_NO_CORRECTION /* a planted mistake: the uncorrected product */
  return q0;
#endif
  return r != r ? q0 : q1;
}

typedef struct {
  int mode; /* 0 bf16, 1 f16, 2 f32 */
  uint32_t t0, t1, stride;
  uint64_t seed;
  long n, bad;
} job;

static int check(job* j, float z, float t, float y) {
  const float a = z / t, b = fast_div(z, t, y);
  j->n++;
  if (f2u(a) != f2u(b) && !(a == 0.0f && b == 0.0f)) {
    if (j->bad < 4) printf("mismatch mode %d z=%a T=%a z/T=%a fast=%a\n", j->mode, z, t, a, b);
    j->bad++;
    return 1;
  }
  return 0;
}

static uint64_t next(uint64_t* s) { /* splitmix64 */
  uint64_t z = (*s += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

static void* run(void* arg) {
  job* j = (job*)arg;
  if (j->mode < 2) {
    for (uint32_t ti = j->t0; ti < j->t1; ti += j->stride) {
      const float t = j->mode == 0 ? u2f(ti << 16) : h2f((uint16_t)ti);
      if (!t_in_range(t)) continue;
      const float y = 1.0f / t;
      for (uint32_t zi = 0; zi < 65536; ++zi) {
        const float z = j->mode == 0 ? u2f(zi << 16) : h2f((uint16_t)zi);
        if (z != z || !z_in_range(z)) continue;
        check(j, z, t, y);
      }
    }
  } else {
    uint64_t s = j->seed;
    for (uint32_t i = j->t0; i < j->t1; ++i) {
      const uint64_t a = next(&s), b = next(&s);
      /* exponent field 31..226 covers [2^-96, 2^100); T's 103..151 covers [2^-24, 2^24] */
      const uint32_t ez = 31u + (uint32_t)(a % 196u), et = 103u + (uint32_t)(b % 49u);
      float z = u2f(((uint32_t)(a >> 32) & 0x80000000u) | (ez << 23) | ((uint32_t)(a >> 8) & 0x7fffffu));
      float t = u2f((et << 23) | ((uint32_t)(b >> 8) & 0x7fffffu));
      if (!t_in_range(t)) t = 1.0f;
      const float y = 1.0f / t;
      check(j, z, t, y);
      /* the same T at the range edges of z */
      if ((i & 1023u) == 0) {
        check(j, 0x1p-96f, t, y);
        check(j, -0x1.fffffep+99f, t, y);
        check(j, INFINITY, t, y);
        check(j, 0.0f, t, y);
      }
    }
  }
  return NULL;
}

int main(int argc, char** argv) {
  const uint32_t f16_stride = argc > 1 ? (uint32_t)atoi(argv[1]) : 5;
  const uint32_t n32 = argc > 2 ? (uint32_t)atoi(argv[2]) : 40000000u;
  long n = 0, bad = 0;
  for (int mode = 0; mode < 3; ++mode) {
    job js[NTHREADS];
    pthread_t th[NTHREADS];
    for (int i = 0; i < NTHREADS; ++i) {
      memset(&js[i], 0, sizeof js[i]);
      js[i].mode = mode;
      if (mode < 2) {
        /* positive T bit patterns only: 0x0000..0x7fff */
        js[i].t0 = (uint32_t)i * (mode == 0 ? 1u : f16_stride);
        js[i].t1 = 0x8000u;
        js[i].stride = NTHREADS * (mode == 0 ? 1u : f16_stride);
      } else {
        js[i].t0 = (uint32_t)((uint64_t)n32 * i / NTHREADS);
        js[i].t1 = (uint32_t)((uint64_t)n32 * (i + 1) / NTHREADS);
        js[i].seed = 0x5eed0000ull + (uint64_t)i;
      }
      pthread_create(&th[i], NULL, run, &js[i]);
    }
    for (int i = 0; i < NTHREADS; ++i) {
      pthread_join(th[i], NULL);
      n += js[i].n;
      bad += js[i].bad;
    }
  }
  printf("cases %ld mismatches %ld\n", n, bad);
  return bad ? 1 : 0;
}
