// Gated-DeltaNet input stage: 4-tap causal conv + SiLU, L2 norm of the q/k heads, gates; fused for decode
// (gdn_conv_l2, T <= 4 with state snapshots) and prefill (gdn_conv_prefill, M tokens, state plane flip), plus the
// unfused twins gdn_conv / gdn_gates / l2norm_heads.
//
// Fused layout: 32 lanes (half a wave) per (head of 128 channels, token or chunk of tokens). Lane p owns the
// channels v + 32k, k = 0..3, of the head, with v = (p & 24) | quad_of_lane(p & 7): the reference's L2-norm lane v
// (src/ops.cu:318-330, 442-446: lane v sums y[v]^2, y[v+32]^2, y[v+64]^2, y[v+96]^2 in that order, then the xor
// butterfly) is then this lane, the sum is in-lane, and the butterfly's xor 16, 8, 4, 2, 1 are lane xor 16, 8, 7,
// 2, 1. Each of the four channel loads / stores of a token covers 128 contiguous bytes over the 32 lanes. In prefill
// the conv window of the last three inputs stays in registers while the lanes walk the span's tokens.
#include "q27h_device.h"
#include "q27h_internal.h"

#ifndef Q27H_GDN_SPAN
#define Q27H_GDN_SPAN 4
#endif

namespace q27h {
namespace {

#ifndef Q27H_NT_GDN
#define Q27H_NT_GDN 1
#endif
constexpr bool kGdnNT = Q27H_NT_GDN;  // nontemporal stores of the prefill conv output

__device__ __forceinline__ float conv4(float s0, float s1, float s2, float xn, const float (&w)[4]) {
  float sum = 0.0f;  // src/ops.cu:419-423: sum = 0; sum += s0 w0; sum += s1 w1; sum += s2 w2; sum += x w3
  sum += s0 * w[0];
  sum += s1 * w[1];
  sum += s2 * w[2];
  sum += xn * w[3];
  return sum;
}

// L2 norm of one 128-channel head held by a 32-lane half, out[k] = channel v + 32k of lane p (layout above).
// Q27H_CONV_RSQ = 1 (the default): the prefill conv's tolerance mode takes the L2 scale from the hardware reciprocal
// square root (within one ulp) instead of the correctly rounded 1 / sqrtf (a chain of about 26 instructions per token
// on each lane of a normed head); measured together with the lean SiLU (Q27H_SILU_LEAN, q27h_device.h): 34.8-35.4
// against 35.9-36.2 us per launch. The exact mode and the decode conv keep 1 / sqrtf.
#ifndef Q27H_CONV_RSQ
#define Q27H_CONV_RSQ 1
#endif
template <bool RSQ = false>
__device__ __forceinline__ void l2_head_lanes(float (&out)[4], float eps) {
  float acc = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; k++) acc += out[k] * out[k];
  acc += lane_xor<16>(acc);
  acc += lane_xor<8>(acc);
  acc += lane_xor<7>(acc);
  acc += lane_xor<2>(acc);
  acc += lane_xor<1>(acc);
  const float scale = RSQ ? __builtin_amdgcn_rsqf(acc / 128.0f + eps / 128.0f)
                          : 1.0f / __builtin_sqrtf(acc / 128.0f + eps / 128.0f);
  const float post = 1.0f / __builtin_sqrtf(128.0f);
#pragma unroll
  for (int k = 0; k < 4; k++) out[k] = (out[k] * scale) * post;
}

// The reference L2 lane held by lane p of a 32-lane half (see the layout note at the top of the file).
__device__ __forceinline__ int l2_lane(int p) { return (p & 24) | quad_of_lane(p & 7); }

__device__ __forceinline__ void gate_one(const float* __restrict__ a, const float* __restrict__ b,
                                         const float* __restrict__ ssm_a, const float* __restrict__ dt_bias,
                                         float* __restrict__ g, float* __restrict__ beta, int t, int H, int hv) {
  const size_t i = (size_t)t * H + hv;
  beta[i] = q27_sigmoid(b[i]);
  g[i] = q27_softplus(a[i] + dt_bias[hv]) * ssm_a[hv];
}

// Prefill: 32 lanes per (head of 128 channels, span of SPAN tokens), a workgroup = 8 neighbouring heads of one span.
// Each XCD runs its share of the tiles in span-major order (the head groups of a span are neighbouring workgroups),
// so the workgroups in flight read and write whole 40 KB rows of the [M][C] arrays: reading 4 KB column pieces of
// many rows instead, as a group-major order does, costs 13% of the bandwidth (measured with a copy of the same shape). Every row of the span
// and the 3-row window before it are loaded up front, then the tokens are computed in order with the window kept in
// registers. The gates (sigmoid / softplus of the H value heads of every token) are not evaluated by the conv lanes:
// the first `gate_blocks` workgroups of the grid take one (token, value head) per lane. Workgroups that walk 16-64
// consecutive tokens of a head group (the window carried in registers, the next span's rows prefetched) measured
// slower: 41-54 against 37.4 us at M = 2048. Spans of 4 tokens (64 VGPRs, 8 waves per SIMD) measured 37.2 us against
// 39.2 / 37.3 / 37.9 us for spans of 3 / 5 / 8 and 10.43-10.46 against 10.47-10.54 ms per prefill pass for 8; the
// token loop without a branch per token (the out-of-range silu redone after the stores) measured the same (37.1 us).
// FAST: the SiLU on the hardware exp2 and reciprocal (q27_silu_tol_n) and the L2 scale on the hardware rsq, within
// the path's fp32 tolerance (1e-5 relative) instead of the checker's bits. The SiLU with a rounding term and a Newton step
// (silu_tol, a few ulps) measured 35.6-36.0 against 37.3-37.4 us for the exact one at M = 2048; without both
// refinements and with the rsq scale 34.8-35.4 against 35.9-36.2 us. The same kernel with no SiLU at all ran
// 34.7-35.0 us, so what remains above a copy of its access shape is the conv, the L2 norm and the stream itself.
template <int SPAN, bool FAST>
__global__ void __launch_bounds__(256) gdn_conv_prefill_kernel(const float* __restrict__ x, const float* __restrict__ cw,
                                                               float* __restrict__ planes, const int* __restrict__ in_plane,
                                                               float* __restrict__ y, int C, int T, int n_norm_heads,
                                                               float eps, const float* __restrict__ a,
                                                               const float* __restrict__ b, const float* __restrict__ ssm_a,
                                                               const float* __restrict__ dt_bias, float* __restrict__ g,
                                                               float* __restrict__ beta, int H, int nspans, int gate_blocks) {
  static_assert(SPAN >= 3, "a span covers the 3-input window");
  if ((int)blockIdx.x < gate_blocks) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < T * H) gate_one(a, b, ssm_a, dt_bias, g, beta, i / H, H, i % H);
    return;
  }
  const int nheads = C / 128;
  const int ngroups = (nheads + 7) / 8;
  // workgroups are handed to the 8 XCDs round-robin, so the workgroups with one value x of bi % 8 share an XCD; they
  // take the tiles [x tpx, (x + 1) tpx) in span-major order, and the window rows of a span were loaded by the span
  // before it on the same XCD (L2 hits)
  const int ntiles = ngroups * nspans, tpx = (ntiles + 7) / 8, bi = blockIdx.x - gate_blocks;
  const int tile = (bi & 7) * tpx + (bi >> 3);
  if (tile >= ntiles) return;
  const int group = tile % ngroups, sp = tile / ngroups;
  const int head = group * 8 + (threadIdx.x >> 5);
  if (head >= nheads) return;  // whole halves leave together
  const int p = threadIdx.x & 31;
  const int cb = head * 128 + l2_lane(p);  // channels cb + 32k
  const int t0 = sp * SPAN, t1 = min(T, t0 + SPAN);
  float xr[SPAN][4];
#pragma unroll
  for (int i = 0; i < SPAN; i++) {
    if (t0 + i < t1) {
#pragma unroll
      for (int k = 0; k < 4; k++) xr[i][k] = x[(size_t)(t0 + i) * C + cb + 32 * k];
    }
  }
  // conv window: s0, s1, s2 = inputs t0-3, t0-2, t0-1 (state plane `pin` before the batch)
  float s0[4], s1[4], s2[4];
  if (t0 == 0) {
    const int pin = *in_plane;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const float* st = planes + ((size_t)pin * C + cb + 32 * k) * 3;
      s0[k] = st[0]; s1[k] = st[1]; s2[k] = st[2];
    }
  } else {
#pragma unroll
    for (int k = 0; k < 4; k++) {
      s0[k] = x[(size_t)(t0 - 3) * C + cb + 32 * k];
      s1[k] = x[(size_t)(t0 - 2) * C + cb + 32 * k];
      s2[k] = x[(size_t)(t0 - 1) * C + cb + 32 * k];
    }
  }
  float w[4][4];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const float4 wv = ld4(cw + 4 * (size_t)(cb + 32 * k));
    w[k][0] = wv.x; w[k][1] = wv.y; w[k][2] = wv.z; w[k][3] = wv.w;
  }
  loads_issued();
  const bool norm = head < n_norm_heads;
#pragma unroll
  for (int i = 0; i < SPAN; i++) {
    const int t = t0 + i;
    if (t >= t1) break;
    float cv[4], cur[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      cv[k] = conv4(s0[k], s1[k], s2[k], xr[i][k], w[k]);
      s0[k] = s1[k]; s1[k] = s2[k]; s2[k] = xr[i][k];
    }
    if constexpr (FAST) q27_silu_tol_n(cv, cur);
    else q27_silu_n(cv, cur);
    if (norm) l2_head_lanes<FAST && Q27H_CONV_RSQ>(cur, eps);
    float* yr = y + (size_t)t * C + cb;
#pragma unroll
    for (int k = 0; k < 4; k++) st_f32<kGdnNT>(yr + 32 * k, cur[k]);
  }
  if (t1 == T) {  // state after the batch: inputs T-3 .. T-1 (from the old state when T < 3)
    const int pin = *in_plane;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      float* o = planes + ((size_t)(pin == 0 ? 1 : 0) * C + cb + 32 * k) * 3;
      o[0] = s0[k]; o[1] = s1[k]; o[2] = s2[k];
    }
  }
}

// Decode (T <= 4, src/ops.cu:288-338): one workgroup per head, 32 lanes per token, so the T tokens run side by side,
// and a third wave that evaluates the head's T gates (a serial chain of exp, division and log that, on a lane of the
// conv waves, added 0.6 us to a 4.1 us node). Token t's window is inputs t-3 .. t-1 (the state plane `pin` for negative ones); snapshot plane t
// receives inputs t-2 .. t. Planes are read before the barrier and written after it, because a snapshot may
// overwrite plane `pin` while another token still needs it.
__global__ void __launch_bounds__(192) gdn_conv_decode_kernel(const float* __restrict__ x, const float* __restrict__ cw,
                                                              float* __restrict__ planes, const int* __restrict__ in_plane,
                                                              float* __restrict__ y, int C, int T, int snapshots,
                                                              int n_norm_heads, float eps, const float* __restrict__ a,
                                                              const float* __restrict__ b, const float* __restrict__ ssm_a,
                                                              const float* __restrict__ dt_bias, float* __restrict__ g,
                                                              float* __restrict__ beta, int H) {
  const int head = blockIdx.x;
  if (threadIdx.x >= 128) {  // the gate wave: gate_one of token (lane) for a value head, beside the conv waves
    __syncthreads();         // the conv waves' one barrier (wave-uniform branch, so the counts match)
    const int lane = threadIdx.x - 128;
    if (head >= n_norm_heads && lane < T) gate_one(a, b, ssm_a, dt_bias, g, beta, lane, H, head - n_norm_heads);
    return;
  }
  const int t = threadIdx.x >> 5, p = threadIdx.x & 31;
  const int cb = head * 128 + l2_lane(p);  // channels cb + 32k
  const bool active = t < T;
  const int pin = *in_plane;
  float in[7][4];  // inputs -3 .. 3 of the lane's 4 channels; token t uses in[t .. t+3]
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const float* st = planes + ((size_t)pin * C + cb + 32 * k) * 3;
    in[0][k] = st[0]; in[1][k] = st[1]; in[2][k] = st[2];
  }
  // rows past the batch are loaded from its last row (an address inside x) and never selected: token t's window
  // reads rows <= t < T only. Unconditional loads and the register selects below keep the code free of per-lane
  // branches (the conditional form compiled to a cascade of divergent branches, each waiting on its own loads).
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const int rr = r < T ? r : T - 1;
#pragma unroll
    for (int k = 0; k < 4; k++) in[3 + r][k] = x[(size_t)rr * C + cb + 32 * k];
  }
  float w[4][4];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const float4 wv = ld4(cw + 4 * (size_t)(cb + 32 * k));
    w[k][0] = wv.x; w[k][1] = wv.y; w[k][2] = wv.z; w[k][3] = wv.w;
  }
  // window of token t, picked by the two bits of t (selects; a chain of t == c tests becomes a switch, i.e.
  // branches that split the wave)
  const bool b0 = (t & 1) != 0, b1 = (t & 2) != 0;
  auto pick = [&](float a0, float a1, float a2, float a3) {
    const float lo = b0 ? a1 : a0, hi = b0 ? a3 : a2;
    return b1 ? hi : lo;
  };
  float s0[4], s1[4], s2[4], xn[4];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    s0[k] = pick(in[0][k], in[1][k], in[2][k], in[3][k]);
    s1[k] = pick(in[1][k], in[2][k], in[3][k], in[4][k]);
    s2[k] = pick(in[2][k], in[3][k], in[4][k], in[5][k]);
    xn[k] = pick(in[3][k], in[4][k], in[5][k], in[6][k]);
  }
  __syncthreads();  // every plane read of the workgroup is consumed before any snapshot write
  if (!active) return;
  float cv[4], out[4];
#pragma unroll
  for (int k = 0; k < 4; k++) cv[k] = conv4(s0[k], s1[k], s2[k], xn[k], w[k]);
  q27_silu_n(cv, out);
  if (snapshots || t == T - 1) {
#pragma unroll
    for (int k = 0; k < 4; k++) {
      float* o = planes + ((size_t)t * C + cb + 32 * k) * 3;
      o[0] = s1[k]; o[1] = s2[k]; o[2] = xn[k];
    }
  }
  if (head < n_norm_heads) l2_head_lanes(out, eps);
  float* yr = y + (size_t)t * C + cb;
  yr[0] = out[0]; yr[32] = out[1]; yr[64] = out[2]; yr[96] = out[3];
}

// l2norm_heads for n = 128: 8 lanes per (token, head); lane q loads channels 4 quad_of_lane(q) + 32k (k = 0..3),
// i.e. four virtual lanes of the reference warp with their four values in summation order.
__global__ void __launch_bounds__(256) l2norm128_kernel(float* __restrict__ x, int heads, int T, int stride, float eps) {
  const int item = blockIdx.x * 32 + (threadIdx.x >> 3);
  if (item >= heads * T) return;  // whole 8-lane groups leave together
  const int t = item / heads, hd = item % heads;
  float* p = x + (size_t)t * stride + (size_t)hd * 128 + block_offset(threadIdx.x);
  float v[4][4];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const float4 a = ld4(p + 32 * k);
    v[k][0] = a.x; v[k][1] = a.y; v[k][2] = a.z; v[k][3] = a.w;
  }
  float s[4];
#pragma unroll
  for (int c = 0; c < 4; c++) {
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; k++) acc += v[k][c] * v[k][c];
    s[c] = acc;
  }
  const float tot = vwarp_sum4(s);
  const float scale = 1.0f / __builtin_sqrtf(tot / 128.0f + eps / 128.0f);
  const float post = 1.0f / __builtin_sqrtf(128.0f);
#pragma unroll
  for (int k = 0; k < 4; k++)
    st4(p + 32 * k, (v[k][0] * scale) * post, (v[k][1] * scale) * post, (v[k][2] * scale) * post, (v[k][3] * scale) * post);
}

// l2norm_heads for any n (src/ops.cu:434-447 structure): 32 lanes per (token, head).
__global__ void __launch_bounds__(256) l2norm_any_kernel(float* __restrict__ x, int n, int heads, int T, int stride, float eps) {
  const int item = blockIdx.x * 8 + (threadIdx.x >> 5);
  if (item >= heads * T) return;
  const int t = item / heads, hd = item % heads, lane = threadIdx.x & 31;
  float* p = x + (size_t)t * stride + (size_t)hd * n;
  float acc = 0.0f;
  for (int i = lane; i < n; i += 32) acc += p[i] * p[i];
  acc = warp32_sum(acc);
  const float scale = 1.0f / __builtin_sqrtf(acc / (float)n + eps / (float)n);
  const float post = 1.0f / __builtin_sqrtf((float)n);
  for (int i = lane; i < n; i += 32) p[i] = (p[i] * scale) * post;
}

__global__ void gdn_gates_kernel(const float* a, const float* b, const float* ssm_a, const float* dt_bias, float* g,
                                 float* beta, int H, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  gate_one(a, b, ssm_a, dt_bias, g, beta, i / H, H, i % H);
}

// gdn_conv_kernel (src/ops.cu:407-431): one thread per channel, T tokens.
__global__ void gdn_conv_kernel(const float* __restrict__ x, const float* __restrict__ cw, float* __restrict__ planes,
                                const int* __restrict__ in_plane, float* __restrict__ y, int C, int T, int snapshots) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= C) return;
  const float* st = planes + ((size_t)(*in_plane) * C + c) * 3;
  float s0 = st[0], s1 = st[1], s2 = st[2];
  const float w[4] = {cw[4 * c], cw[4 * c + 1], cw[4 * c + 2], cw[4 * c + 3]};
  for (int t = 0; t < T; t++) {
    const float xn = x[(size_t)t * C + c];
    y[(size_t)t * C + c] = q27_silu(conv4(s0, s1, s2, xn, w));
    s0 = s1; s1 = s2; s2 = xn;
    if (snapshots || t == T - 1) {
      float* o = planes + ((size_t)t * C + c) * 3;
      o[0] = s0; o[1] = s1; o[2] = s2;
    }
  }
}

__global__ void flip_plane_kernel(int* p) { *p = *p == 0 ? 1 : 0; }
__global__ void flip_plane_to_kernel(int* dst, const int* src) { *dst = *src == 0 ? 1 : 0; }

int check_fused(const char* fn, const float* x, const float* w, const float* planes, const int* in_plane, const float* y,
                int C, int T, int n_norm_heads, int H, const float* a, const float* b, const float* ssm_a,
                const float* dt_bias, const float* g, const float* beta) {
  if (C <= 0 || C % 128 || C / 128 - n_norm_heads != H || n_norm_heads < 0 || T < 0)
    return fail(Q27H_ERR_SHAPE, std::string(fn) + ": bad shape");
  if (!x || !w || !planes || !in_plane || !y) return fail(Q27H_ERR_ARG, std::string(fn) + ": null pointer");
  if (H > 0 && (!a || !b || !ssm_a || !dt_bias || !g || !beta)) return fail(Q27H_ERR_ARG, std::string(fn) + ": null gate pointer");
  if (!aligned16(x) || !aligned16(w) || !aligned16(planes) || !aligned16(y))
    return fail(Q27H_ERR_ARG, std::string(fn) + ": x, w, planes, y need 16-byte alignment");
  return Q27H_OK;
}

}  // namespace
}  // namespace q27h

using namespace q27h;

extern "C" int q27h_gdn_conv_l2(const float* x, const float* w, float* planes, const int* in_plane, float* y, int C, int T,
                                int snapshots, int n_norm_heads, float eps, const float* a, const float* b,
                                const float* ssm_a, const float* dt_bias, float* g, float* beta, int H, q27h_stream_t s,
                                const void* pf, size_t pf_bytes) {
  (void)pf;
  (void)pf_bytes;
  if (int e = check_fused("gdn_conv_l2", x, w, planes, in_plane, y, C, T, n_norm_heads, H, a, b, ssm_a, dt_bias, g, beta))
    return e;
  if (T > 4) return fail(Q27H_ERR_SHAPE, "gdn_conv_l2: T must be <= 4 (4 state planes)");
  if (T == 0) return Q27H_OK;
  hipLaunchKernelGGL(gdn_conv_decode_kernel, dim3(C / 128), dim3(192), 0, stream_of(s), x, w, planes, in_plane, y, C, T,
                     snapshots, n_norm_heads, eps, a, b, ssm_a, dt_bias, g, beta, H);
  return check_launch("gdn_conv_l2");
}

extern "C" int q27h_gdn_conv_prefill(const float* x, const float* w, float* planes, const int* in_plane, float* y, int C,
                                     int M, int n_norm_heads, float eps, const float* a, const float* b, const float* ssm_a,
                                     const float* dt_bias, float* g, float* beta, int H, q27h_stream_t s) {
  if (int e = check_fused("gdn_conv_prefill", x, w, planes, in_plane, y, C, M, n_norm_heads, H, a, b, ssm_a, dt_bias, g, beta))
    return e;
  if (M == 0) return Q27H_OK;
  constexpr int span = Q27H_GDN_SPAN;  // tokens per half-wave
  const int gate_blocks = (int)(((long)M * H + 255) / 256);
  const int nspans = (M + span - 1) / span;
  const long tiles = ((long)((C / 128 + 7) / 8) * nspans + 7) / 8 * 8;  // a whole number of tiles per XCD
  // the SiLU and L2 scale of the conv output: within the fp32 tolerance unless the process asked for the checker's bits
  // (q27h_gdn_prefill_exact, read here when the launch is enqueued)
  if (gdn_prefill_exact_mode())
    hipLaunchKernelGGL((gdn_conv_prefill_kernel<span, false>), dim3((unsigned)(tiles + gate_blocks)), dim3(256), 0,
                       stream_of(s), x, w, planes, in_plane, y, C, M, n_norm_heads, eps, a, b, ssm_a, dt_bias, g, beta, H,
                       nspans, gate_blocks);
  else
    hipLaunchKernelGGL((gdn_conv_prefill_kernel<span, true>), dim3((unsigned)(tiles + gate_blocks)), dim3(256), 0,
                       stream_of(s), x, w, planes, in_plane, y, C, M, n_norm_heads, eps, a, b, ssm_a, dt_bias, g, beta, H,
                       nspans, gate_blocks);
  return check_launch("gdn_conv_prefill");
}

extern "C" int q27h_l2norm_heads(float* x, int n, int heads, int T, int stride, float eps, q27h_stream_t s) {
  if (n <= 0 || heads < 0 || T < 0) return fail(Q27H_ERR_SHAPE, "l2norm_heads: bad shape");
  if (!x) return fail(Q27H_ERR_ARG, "l2norm_heads: null pointer");
  const long items = (long)heads * T;
  if (items == 0) return Q27H_OK;
  if (n == 128 && stride % 4 == 0 && aligned16(x))
    hipLaunchKernelGGL(l2norm128_kernel, dim3((unsigned)((items + 31) / 32)), dim3(256), 0, stream_of(s), x, heads, T, stride,
                       eps);
  else
    hipLaunchKernelGGL(l2norm_any_kernel, dim3((unsigned)((items + 7) / 8)), dim3(256), 0, stream_of(s), x, n, heads, T, stride,
                       eps);
  return check_launch("l2norm_heads");
}

namespace q27h {
namespace {
// gemv_bf16_pair (src/ops.cu:377-393): y[t][row] of the two bf16 matrices [Wa; Wb] (N rows each, K columns) in the
// reference's arithmetic: 256 virtual threads, thread v adds (w[k] x[k] + w[k + 1] x[k + 1]) for k = 2v + 512 j in
// order, then block_sum (warp xor butterflies, 8 warp sums, second butterfly). One wave per (row, token): lane l holds
// the virtual threads 32 (l / 8) + 4 quad_of_lane(l % 8) + c, c = 0..3, so its four pairs are 8 consecutive values
// (one 16-byte load of weights per step) and the warp butterfly is lane xor 7, 2, 1 plus the lane's own pairs; the
// 8 warp sums live in the 8 lane groups and meet through lane xor 32, 16, 8 (the second butterfly's xor 4, 2, 1;
// its xor 16 and 8 only add the zero entries).
constexpr int kPairU = 10;  // steps of 512 weights in flight per lane
__global__ void __launch_bounds__(256) gemv_bf16_pair_kernel(const uint16_t* __restrict__ Wa, const uint16_t* __restrict__ Wb,
                                                             const float* __restrict__ x, float* __restrict__ ya,
                                                             float* __restrict__ yb, int N, int K, int T) {
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wave >= 2 * N * T) return;  // whole waves
  const int row = wave % (2 * N), t = wave / (2 * N);
  const int l = threadIdx.x & 63;
  const uint16_t* w = row < N ? Wa + (size_t)row * K : Wb + (size_t)(row - N) * K;
  const float* xt = x + (size_t)t * K;
  const int k0 = 2 * (32 * (l >> 3) + 4 * quad_of_lane(l & 7));
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  // kPairU steps of 512 weights (all of a 5120-wide row) are requested before the first is used, then added in k
  // order: weights from HBM cost one memory round trip per batch instead of one per step. 48 x 5120, graph of 320
  // launches over distinct weight pairs: 7.13 -> 4.01 us (T = 1), 6.85 -> 3.98 us (T = 4); one cached pair 3.20 ->
  // 3.02 us. The sums and their order are unchanged.
  for (int kb = k0; kb < K; kb += 512 * kPairU) {
    uint4 wv[kPairU];
    float4 xa[kPairU], xb[kPairU];
#pragma unroll
    for (int u = 0; u < kPairU; u++) {
      const int k = kb + 512 * u;
      if (k < K) {
        wv[u] = *(const uint4*)(w + k);
        xa[u] = ld4(xt + k);
        xb[u] = ld4(xt + k + 4);
      }
    }
#pragma unroll
    for (int u = 0; u < kPairU; u++) {
      if (kb + 512 * u >= K) break;
      const uint32_t ww[4] = {wv[u].x, wv[u].y, wv[u].z, wv[u].w};
      const float xx[8] = {xa[u].x, xa[u].y, xa[u].z, xa[u].w, xb[u].x, xb[u].y, xb[u].z, xb[u].w};
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const float w0 = bf16_to_f((uint16_t)(ww[c] & 0xffff)), w1 = bf16_to_f((uint16_t)(ww[c] >> 16));
        acc[c] = acc[c] + (w0 * xx[2 * c] + w1 * xx[2 * c + 1]);
      }
    }
  }
  float v = vwarp_sum4(acc);
  v = (v + 0.0f) + 0.0f;  // the second butterfly's xor 16 and xor 8 steps (zero entries)
  v += lane_xor32(v);
  v += lane_xor<16>(v);
  v += lane_xor<8>(v);
  if (l == 0) (row < N ? ya[(size_t)t * N + row] : yb[(size_t)t * N + row - N]) = v;
}
}  // namespace
}  // namespace q27h

extern "C" int q27h_gemv_bf16_pair(const uint16_t* Wa, const uint16_t* Wb, const float* x, float* ya, float* yb, int N,
                                   int K, int T, q27h_stream_t s) {
  if (N <= 0 || K <= 0 || K % 8 || T < 0) return fail(Q27H_ERR_SHAPE, "gemv_bf16_pair: bad shape (K % 8 == 0)");
  if (T == 0) return Q27H_OK;
  if (!Wa || !Wb || !x || !ya || !yb) return fail(Q27H_ERR_ARG, "gemv_bf16_pair: null pointer");
  if (!aligned16(Wa) || !aligned16(Wb) || !aligned16(x))
    return fail(Q27H_ERR_ARG, "gemv_bf16_pair: Wa, Wb and x need 16-byte alignment");
  const int waves = 2 * N * T;
  hipLaunchKernelGGL(gemv_bf16_pair_kernel, dim3((waves + 3) / 4), dim3(256), 0, stream_of(s), Wa, Wb, x, ya, yb, N, K, T);
  return check_launch("gemv_bf16_pair");
}

extern "C" int q27h_gdn_gates(const float* a, const float* b, const float* ssm_a, const float* dt_bias, float* g, float* beta,
                              int H, int T, q27h_stream_t s) {
  if (H <= 0 || T < 0) return fail(Q27H_ERR_SHAPE, "gdn_gates: bad shape");
  if (T == 0) return Q27H_OK;
  hipLaunchKernelGGL(gdn_gates_kernel, dim3((H * T + 127) / 128), dim3(128), 0, stream_of(s), a, b, ssm_a, dt_bias, g, beta, H,
                     H * T);
  return check_launch("gdn_gates");
}

extern "C" int q27h_gdn_conv(const float* x, const float* w, float* planes, const int* in_plane, float* y, int C, int T,
                             int snapshots, q27h_stream_t s) {
  if (C <= 0 || T < 0 || T > 4) return fail(Q27H_ERR_SHAPE, "gdn_conv: bad shape (T <= 4)");
  if (T == 0) return Q27H_OK;
  hipLaunchKernelGGL(gdn_conv_kernel, dim3((C + 255) / 256), dim3(256), 0, stream_of(s), x, w, planes, in_plane, y, C, T,
                     snapshots);
  return check_launch("gdn_conv");
}

extern "C" int q27h_gdn_flip_plane(int* plane, q27h_stream_t s) {
  if (!plane) return fail(Q27H_ERR_ARG, "gdn_flip_plane: null pointer");
  hipLaunchKernelGGL(flip_plane_kernel, dim3(1), dim3(1), 0, stream_of(s), plane);
  return check_launch("gdn_flip_plane");
}

extern "C" int q27h_flip_plane_to(int* dst, const int* src, q27h_stream_t s) {
  if (!dst || !src) return fail(Q27H_ERR_ARG, "flip_plane_to: null pointer");
  hipLaunchKernelGGL(flip_plane_to_kernel, dim3(1), dim3(1), 0, stream_of(s), dst, src);
  return check_launch("flip_plane_to");
}
