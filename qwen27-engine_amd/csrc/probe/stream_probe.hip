// Measurement only (bench.py), not part of the fused-op library: streaming kernels that move the same bytes as a fused
// op with no arithmetic, to measure what HBM delivers for that op's mix of reads and writes on the box at hand.
//
// q27p_flat: n values; thread t of a 256-thread workgroup handles 4 consecutive values per 1024-value chunk (the
// layout of the fused ops). Per value it reads nin f32 streams (16-byte nontemporal loads), writes nout f32 streams
// (16-byte stores; rmw: the first output is the first input, written in place), and, when q is set, the q8_1 output
// of the fused ops: one int8 per value, one f32 per 32 values (d) and, when s is set, one f32 per 16 values.
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

template <int NIN, int NOUT>
__global__ void __launch_bounds__(256) flat_probe(const float* __restrict__ a, const float* __restrict__ b,
                                                  float* __restrict__ o0, float* __restrict__ o1, int8_t* __restrict__ q,
                                                  float* __restrict__ d, float* __restrict__ s, size_t n) {
  const size_t i = (size_t)blockIdx.x * 1024 + 4 * threadIdx.x;
  if (i >= n) return;
  v4f v = {0.f, 0.f, 0.f, 0.f};
  if (NIN >= 1) v = __builtin_nontemporal_load((const v4f*)(a + i));
  if (NIN >= 2) v += __builtin_nontemporal_load((const v4f*)(b + i));
  if (NOUT >= 1) *(v4f*)(o0 + i) = v;
  if (NOUT >= 2) *(v4f*)(o1 + i) = v * 2.0f;
  if (q) {
    *(uint32_t*)(q + i) = (uint32_t)(int)v.x;
    if ((threadIdx.x & 7) == 0) d[i / 32] = v.y;
    if (s && (threadIdx.x & 3) == 0) s[i / 16] = v.z;
  }
}

}  // namespace

extern "C" int q27p_flat(const float* a, const float* b, float* o0, float* o1, int8_t* q, float* d, float* s, size_t n, int nin,
                         int nout, void* stream) {
  if (n % 1024 || nin < 0 || nin > 2 || nout < 0 || nout > 2) return -1;
  const dim3 grid((unsigned)(n / 1024)), block(256);
  hipStream_t st = (hipStream_t)stream;
#define Q27P_CASE(I, O)                                                                                   \
  if (nin == I && nout == O) {                                                                            \
    hipLaunchKernelGGL((flat_probe<I, O>), grid, block, 0, st, a, b, o0, o1, q, d, s, n);                 \
    return hipGetLastError() == hipSuccess ? 0 : -2;                                                      \
  }
  Q27P_CASE(0, 1) Q27P_CASE(0, 2) Q27P_CASE(1, 0) Q27P_CASE(1, 1) Q27P_CASE(1, 2) Q27P_CASE(2, 0) Q27P_CASE(2, 1) Q27P_CASE(2, 2)
#undef Q27P_CASE
  return -1;
}
