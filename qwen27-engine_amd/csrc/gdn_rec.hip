// Gated-DeltaNet recurrence (the delta rule) over T tokens for H value heads of 128 x 128 f32 state (gdn_step,
// src/ops.h:40-45, src/ops.cu:449-572, 784-793). Per head h (key head kh = h % HK), value column col and token t:
//   kv    = sum_i S[i][col] k[i]
//   delta = (v[col] - e^g kv) beta
//   S[i][col] = e^g S[i][col] + k[i] delta
//   o[t][h][col] = (sum_i S[i][col] q[i]) scale
// State planes [4][H][128 col][128 i] (column col of S contiguous). Decode (flip = false): read plane *in_plane,
// write plane t after token t when `snapshots` (else only after the last token, to plane T - 1). Prefill (flip =
// true, any T): no snapshots; the final state goes to plane (*in_plane == 0 ? 1 : 0).
//
// gfx950 layout: 16 lanes per column, lane part p holds S[8p .. 8p + 7][col] in registers for the whole sequence; a
// 512-thread workgroup = 32 columns of one head (grid H x 4). Per token each lane forms its 8-term partial dot
// products as four interleaved partial sums, (k0 + k1) + (k2 + k3), and the 16 parts are added by an xor butterfly
// (masks 1, 2, 7, 8). q, k of GT tokens (shared by the 32 columns), v, e^g and beta are staged in
// LDS once per GT tokens. The CPU checker restates this order exactly.
#include "q27h_device.h"
#include "q27h_internal.h"

namespace q27h {
namespace {

constexpr int kParts = 16, kEpl = 128 / kParts;  // lanes per column, state elements per lane
constexpr int kCols = 32;                         // columns per workgroup
constexpr int kGT = 32;                           // tokens staged per LDS round

// Sum over the 16 parts of a column (lanes 16c .. 16c + 15): xor butterfly with masks 1, 2, 7, 8, which span lane
// bits 0..3 and are all DPP moves (quad_perm, row_half_mirror, row_ror:8). Each step adds a lane pair's two values,
// so every part ends with the bit-identical sum.
__device__ __forceinline__ float parts_sum(float v) {
  v += lane_xor<1>(v);
  v += lane_xor<2>(v);
  v += lane_xor<7>(v);
  v += lane_xor<8>(v);
  return v;
}

__global__ void __launch_bounds__(kCols * kParts) gdn_rec_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                                 const float* __restrict__ v, int stride,
                                                                 const float* __restrict__ g, const float* __restrict__ beta,
                                                                 float* __restrict__ planes, const int* __restrict__ in_plane,
                                                                 float* __restrict__ o, int H, int HK, int T, float scale,
                                                                 int snapshots, int flip) {
  __shared__ __align__(16) float sq[kGT][128];
  __shared__ __align__(16) float sk[kGT][128];
  __shared__ float sv[kGT][kCols];
  __shared__ float sg[kGT], sb[kGT];
  const int h = blockIdx.x, kh = h % HK;
  const int tid = threadIdx.x, p = tid & (kParts - 1), cl = tid / kParts, col = blockIdx.y * kCols + cl;
  const size_t plane_sz = (size_t)H * 128 * 128;
  const int pin = *in_plane;
  const size_t soff = ((size_t)h * 128 + col) * 128 + kEpl * p;
  float s[kEpl];
  {
    const float* src = planes + (size_t)pin * plane_sz + soff;
    const float4 a = ld4(src), b = ld4(src + 4);
    s[0] = a.x; s[1] = a.y; s[2] = a.z; s[3] = a.w; s[4] = b.x; s[5] = b.y; s[6] = b.z; s[7] = b.w;
  }
  const int out_plane = flip ? (pin == 0 ? 1 : 0) : T - 1;
  for (int t0 = 0; t0 < T; t0 += kGT) {
    const int nt = min(kGT, T - t0);
    __syncthreads();  // the previous round's reads of the staging buffers are done
    for (int i = tid; i < nt * 32; i += kCols * kParts) {  // 32 float4 per token per vector
      const int t = i >> 5, e4 = (i & 31) * 4;
      *(float4*)&sq[t][e4] = ld4(q + (size_t)(t0 + t) * stride + kh * 128 + e4);
      *(float4*)&sk[t][e4] = ld4(k + (size_t)(t0 + t) * stride + kh * 128 + e4);
    }
    for (int i = tid; i < nt * kCols; i += kCols * kParts) {
      const int t = i / kCols, c = i % kCols;
      sv[t][c] = v[(size_t)(t0 + t) * stride + h * 128 + blockIdx.y * kCols + c];
    }
    if (tid < nt) {
      sg[tid] = q27_expf(g[(size_t)(t0 + tid) * H + h]);
      sb[tid] = beta[(size_t)(t0 + tid) * H + h];
    }
    __syncthreads();
    for (int tt = 0; tt < nt; tt++) {
      const float4 k0 = *(const float4*)&sk[tt][kEpl * p], k1 = *(const float4*)&sk[tt][kEpl * p + 4];
      const float4 q0 = *(const float4*)&sq[tt][kEpl * p], q1 = *(const float4*)&sq[tt][kEpl * p + 4];
      const float kr[kEpl] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
      const float qr[kEpl] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
      float kq[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int i = 0; i < kEpl; i++) kq[i & 3] += s[i] * kr[i];
      const float kv = parts_sum((kq[0] + kq[1]) + (kq[2] + kq[3]));
      const float gv = sg[tt];
      const float delta = (sv[tt][cl] - gv * kv) * sb[tt];
      float aq[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int i = 0; i < kEpl; i++) {
        s[i] = gv * s[i] + kr[i] * delta;
        aq[i & 3] += s[i] * qr[i];
      }
      const float at = parts_sum((aq[0] + aq[1]) + (aq[2] + aq[3]));
      const int t = t0 + tt;
      if (p == 0) o[((size_t)t * H + h) * 128 + col] = at * scale;
      if (!flip && snapshots && t < T - 1) {
        float* W = planes + (size_t)t * plane_sz + soff;
        st4(W, s[0], s[1], s[2], s[3]);
        st4(W + 4, s[4], s[5], s[6], s[7]);
      }
    }
  }
  float* W = planes + (size_t)out_plane * plane_sz + soff;
  st4(W, s[0], s[1], s[2], s[3]);
  st4(W + 4, s[4], s[5], s[6], s[7]);
}

}  // namespace
}  // namespace q27h

using namespace q27h;

extern "C" int q27h_gdn_step(const float* q, const float* k, const float* v, int stride, const float* g, const float* beta,
                             float* planes, const int* in_plane, float* o, int H, int HK, int T, float scale, int snapshots,
                             q27h_stream_t s, int flip) {
  if (H <= 0 || HK <= 0 || T < 0 || stride < 128 || stride % 4) return fail(Q27H_ERR_SHAPE, "gdn_step: bad shape");
  if (!flip && T > 4) return fail(Q27H_ERR_SHAPE, "gdn_step: T must be <= 4 without flip (4 state planes)");
  if (T == 0) return Q27H_OK;
  if (!q || !k || !v || !g || !beta || !planes || !in_plane || !o) return fail(Q27H_ERR_ARG, "gdn_step: null pointer");
  if (!aligned16(q) || !aligned16(k) || !aligned16(planes))
    return fail(Q27H_ERR_ARG, "gdn_step: q, k and planes need 16-byte alignment");
  hipLaunchKernelGGL(gdn_rec_kernel, dim3(H, 128 / kCols), dim3(kCols * kParts), 0, stream_of(s), q, k, v, stride, g, beta,
                     planes, in_plane, o, H, HK, T, scale, snapshots, flip);
  return check_launch("gdn_step");
}
