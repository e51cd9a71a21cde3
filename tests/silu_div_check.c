/* Host check of the device's silu quotient (div_silu in qwen27-engine_amd/csrc/q27h_device.h): for float x with
 * 2^-60 <= |x| <= 60, d = 1 + expf_core(-x) (the device's exp sequence), and the hardware reciprocal y0 modelled as
 * RN(1/d) moved by -1, 0 or +1 ulp, the sequence y = fma(fma(-d, y0, 1), y0, y0), q0 = x y,
 * q1 = fma(fma(-d, q0, x), y, q0) must equal the IEEE quotient x / d; the two-correction form of the IEEE sequence
 * (q2 = fma(fma(-d, q1, x), y, q1)) is checked beside it. Arguments: STRIDE (1 = every float of the range) and the
 * thread count; every x of [2^-26, 2^-20] is always included. Prints one line per (form, reciprocal offset) with the
 * mismatch count and the first mismatching x (hex float). */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static float expf_core(float x) {  /* q27_expf_core */
  const float k = rintf(x * 1.44269502f);
  float r = fmaf(-k, 0.693145752f, x);
  r = fmaf(-k, 1.42860677e-06f, r);
  float p = 1.98412698e-4f;
  p = fmaf(p, r, 1.38888889e-3f);
  p = fmaf(p, r, 8.33333333e-3f);
  p = fmaf(p, r, 4.16666667e-2f);
  p = fmaf(p, r, 1.66666667e-1f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return ldexpf(p, (int)k);
}

#define MAXT 64
static uint64_t g_stride;
static int g_threads;
static uint64_t bad[MAXT][2][3];
static float first[MAXT][2][3];

static void check(int t, float x) {
  const float d = 1.0f + expf_core(-x);
  const float want = x / d;
  const float rn = (float)(1.0 / (double)d);
  for (int k = 0; k < 3; k++) {
    const float y0 = k == 1 ? rn : nextafterf(rn, k == 0 ? 0.0f : INFINITY);
    const float y = fmaf(fmaf(-d, y0, 1.0f), y0, y0);
    const float q0 = x * y;
    const float q1 = fmaf(fmaf(-d, q0, x), y, q0);
    const float q2 = fmaf(fmaf(-d, q1, x), y, q1);
    if (to_bits(q1) != to_bits(want)) { if (!bad[t][0][k]) first[t][0][k] = x; bad[t][0][k]++; }
    if (to_bits(q2) != to_bits(want)) { if (!bad[t][1][k]) first[t][1][k] = x; bad[t][1][k]++; }
  }
}

static void* run(void* arg) {
  const int t = (int)(long)arg;
  const uint32_t lo = to_bits(0x1p-60f), hi = to_bits(60.0f), blo = to_bits(0x1p-26f), bhi = to_bits(0x1p-20f);
  for (uint64_t u = lo + (uint64_t)t * g_stride; u <= hi; u += (uint64_t)g_threads * g_stride)
    if (u < blo || u > bhi) { check(t, from_bits((uint32_t)u)); check(t, -from_bits((uint32_t)u)); }
  for (uint64_t u = blo + (uint64_t)t; u <= bhi; u += (uint64_t)g_threads) {
    check(t, from_bits((uint32_t)u));
    check(t, -from_bits((uint32_t)u));
  }
  return NULL;
}

int main(int argc, char** argv) {
  g_stride = argc > 1 ? strtoull(argv[1], NULL, 10) : 1;
  g_threads = argc > 2 ? atoi(argv[2]) : 8;
  if (g_stride < 1 || g_threads < 1 || g_threads > MAXT) return 2;
  pthread_t th[MAXT];
  for (long t = 0; t < g_threads; t++) pthread_create(&th[t], NULL, run, (void*)t);
  for (int t = 0; t < g_threads; t++) pthread_join(th[t], NULL);
  for (int f = 0; f < 2; f++)
    for (int k = 0; k < 3; k++) {
      uint64_t n = 0;
      float x0 = 0.0f;
      for (int t = 0; t < g_threads; t++) {
        if (bad[t][f][k] && n == 0) x0 = first[t][f][k];
        n += bad[t][f][k];
      }
      printf("%s %d %llu %a\n", f == 0 ? "one" : "two", k - 1, (unsigned long long)n, x0);
    }
  return 0;
}
