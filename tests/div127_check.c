/* Exhaustive host check of the device's amax / 127 (div127 in qwen27-engine_amd/csrc/q27h_device.h):
 * q0 = a * RN(1/127), r = fma(-127, q0, a), q1 = fma(r, RN(1/127), q0) must equal the IEEE quotient a / 127 for
 * every non-negative finite float a (subnormals included). Prints the number of mismatches (0 expected). */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#define NTHREADS 8
static long bad[NTHREADS];

static void* run(void* arg) {
  const long t = (long)arg;
  const float inv = 1.0f / 127.0f;
  for (uint64_t u = (uint64_t)t; u < 0x7f800000u; u += NTHREADS) {
    const uint32_t bits = (uint32_t)u;
    float a;
    memcpy(&a, &bits, 4);
    const float q0 = a * inv;
    const float r = fmaf(-127.0f, q0, a);
    const float q1 = fmaf(r, inv, q0);
    const float want = a / 127.0f;
    if (memcmp(&q1, &want, 4) != 0) bad[t]++;
  }
  return 0;
}

int main(void) {
  pthread_t th[NTHREADS];
  for (long i = 0; i < NTHREADS; i++) pthread_create(&th[i], 0, run, (void*)i);
  long total = 0;
  for (int i = 0; i < NTHREADS; i++) {
    pthread_join(th[i], 0);
    total += bad[i];
  }
  printf("%ld\n", total);
  return 0;
}
