// The wire formats of the two-card partial-sum exchange (src/prefill.h:34-44, src/prefill.cu:338-370,503-509): bf16
// rows (to_bf16) and q8 rows with error feedback (to_q8_wire). These are the encoders on either side of a2's sum; the
// decoder side is add_norm_rows_q8 (the row engine in norm_q8.hip). Moving the rows between GPUs is not part of this
// library.
//
// q8 wire row (n = 5120 values): n int8 values, then n / qb fp16 scales (qb = 16: "q8b16", qb = 32: "q8"). Per block
// of qb values: y = partial (+ ef unless first), amax = max |y|, d = amax / 127, q = amax == 0 ? 0 : roundf(y / d),
// scale = fp16(d), and ef = y - fp16(d) q (the rounding error carried to the next exchange).
#include <algorithm>

#include "q27h_device.h"
#include "q27h_internal.h"

namespace q27h {
namespace {

// One 256-thread workgroup per row, in the row engine's lane layout (thread t holds the four values at
// 32 (t / 8) + block_offset(t) of each 1024-value slice): a 16-value block is lanes 0..3 or 4..7 of a group of 8,
// a 32-value block the whole group.
template <int QB>
__global__ void __launch_bounds__(256) to_q8_wire_kernel(const float* __restrict__ partial, float* __restrict__ ef, int first,
                                                         uint8_t* __restrict__ wire) {
  constexpr size_t kRb = kRowN + 2 * kRowN / QB;
  const int t = threadIdx.x;
  const size_t row = blockIdx.x;
  const int off = 32 * (t >> 3) + block_offset(t);
  const float* pr = partial + row * kRowN;
  float* er = ef ? ef + row * kRowN : nullptr;
  uint8_t* wr = wire + row * kRb;
  float4 pv[5], ev[5];
#pragma unroll
  for (int k = 0; k < 5; k++) pv[k] = ld4_nt(pr + off + k * 1024);
  if (er && !first) {
#pragma unroll
    for (int k = 0; k < 5; k++) ev[k] = ld4(er + off + k * 1024);
  }
#pragma unroll
  for (int k = 0; k < 5; k++) {
    const int i = off + k * 1024;
    float y[4] = {pv[k].x, pv[k].y, pv[k].z, pv[k].w};
    if (er && !first) {
      y[0] = y[0] + ev[k].x; y[1] = y[1] + ev[k].y; y[2] = y[2] + ev[k].z; y[3] = y[3] + ev[k].w;
    }
    float amax = __builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(y[0]), __builtin_fabsf(y[1])),
                                 __builtin_fmaxf(__builtin_fabsf(y[2]), __builtin_fabsf(y[3])));
    if constexpr (QB == 32) amax = __builtin_fmaxf(amax, lane_xor<7>(amax));
    amax = __builtin_fmaxf(amax, lane_xor<2>(amax));
    amax = __builtin_fmaxf(amax, lane_xor<1>(amax));
    const float d = div127(amax);
    int q[4];
    q8_round_div4(y, d, q);
    st_u32<true>((int8_t*)wr + i, pack4_i8(q[0], q[1], q[2], q[3]));
    const uint16_t dh = f2h_bits(d);
    if ((i & (QB - 1)) == 0) *(uint16_t*)(wr + kRowN + 2 * (i / QB)) = dh;
    if (er) {
      const float df = h2f_bits(dh);
      st4<false>(er + i, y[0] - df * (float)q[0], y[1] - df * (float)q[1], y[2] - df * (float)q[2],
                 y[3] - df * (float)q[3]);
    }
  }
}

// y = bf16(x) (round to nearest even), four values per thread and step where x / y are 16 / 8-byte aligned and
// n % 4 == 0, pairs otherwise.
__device__ __forceinline__ uint32_t bf16x2(float a, float b) {
  return (__builtin_bit_cast(uint32_t, bf16_round(a)) >> 16) | (__builtin_bit_cast(uint32_t, bf16_round(b)) & 0xffff0000u);
}
__global__ void to_bf16_quad_kernel(const float* __restrict__ x, uint16_t* __restrict__ y, size_t nq) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < nq; i += (size_t)gridDim.x * blockDim.x) {
    const float4 v = ld4_nt(x + 4 * i);
    uint2 o;
    o.x = bf16x2(v.x, v.y);
    o.y = bf16x2(v.z, v.w);
    __builtin_nontemporal_store(o.x, (uint32_t*)(y + 4 * i));
    __builtin_nontemporal_store(o.y, (uint32_t*)(y + 4 * i) + 1);
  }
}
__global__ void to_bf16_pair_kernel(const float* __restrict__ x, uint16_t* __restrict__ y, size_t np) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < np; i += (size_t)gridDim.x * blockDim.x)
    *(uint32_t*)(y + 2 * i) = bf16x2(x[2 * i], x[2 * i + 1]);
}

}  // namespace
}  // namespace q27h

using namespace q27h;

extern "C" int q27h_to_q8_wire(const float* partial, float* ef, int first, uint8_t* wire, int n, int M, int qb,
                               q27h_stream_t s) {
  if (n != kRowN) return fail(Q27H_ERR_SHAPE, "to_q8_wire: n must be 5120");
  if (qb != 16 && qb != 32) return fail(Q27H_ERR_SHAPE, "to_q8_wire: qb must be 16 or 32 (the q8 wires)");
  if (M < 0) return fail(Q27H_ERR_SHAPE, "to_q8_wire: M < 0");
  if (M == 0) return Q27H_OK;
  if (!partial || !wire) return fail(Q27H_ERR_ARG, "to_q8_wire: null pointer");
  if (!aligned16(partial) || (ef && !aligned16(ef)) || !aligned16(wire))
    return fail(Q27H_ERR_ARG, "to_q8_wire: partial, ef and wire need 16-byte alignment");
  if (qb == 16)
    hipLaunchKernelGGL(to_q8_wire_kernel<16>, dim3(M), dim3(256), 0, stream_of(s), partial, ef, first, wire);
  else
    hipLaunchKernelGGL(to_q8_wire_kernel<32>, dim3(M), dim3(256), 0, stream_of(s), partial, ef, first, wire);
  return check_launch("to_q8_wire");
}

extern "C" int q27h_to_bf16(const float* x, uint16_t* y, size_t n, q27h_stream_t s) {
  if (n % 2) return fail(Q27H_ERR_SHAPE, "to_bf16: n must be even");
  if (n == 0) return Q27H_OK;
  if (!x || !y) return fail(Q27H_ERR_ARG, "to_bf16: null pointer");
  if (((uintptr_t)x & 7u) || ((uintptr_t)y & 3u)) return fail(Q27H_ERR_ARG, "to_bf16: x needs 8-byte, y 4-byte alignment");
  if (n % 4 == 0 && aligned16(x) && ((uintptr_t)y & 7u) == 0) {
    const size_t nq = n / 4;
    const size_t grid = std::min<size_t>((nq + 255) / 256, 256 * 16);
    hipLaunchKernelGGL(to_bf16_quad_kernel, dim3((unsigned)grid), dim3(256), 0, stream_of(s), x, y, nq);
  } else {
    const size_t np = n / 2;
    const size_t grid = std::min<size_t>((np + 255) / 256, 256 * 16);
    hipLaunchKernelGGL(to_bf16_pair_kernel, dim3((unsigned)grid), dim3(256), 0, stream_of(s), x, y, np);
  }
  return check_launch("to_bf16");
}
