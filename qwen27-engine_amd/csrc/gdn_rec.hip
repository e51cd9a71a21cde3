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
// products as four interleaved fused multiply-add chains, (k0 + k1) + (k2 + k3), and the 16 parts are added by an
// xor butterfly (masks 1, 2, 7, 8); the state update is fma(k, delta, e^g S). q, k of kGT tokens (shared by the
// 32 columns), v, e^g and beta are staged in LDS, double-buffered: the next round's global loads are in flight
// while the current round's tokens run. The CPU checker restates this order exactly. The kernel is bound by VALU
// issue (about 60 instructions per token and wave, two waves per SIMD), not by HBM.
#include <atomic>

#include "q27h_device.h"
#include "q27h_internal.h"

namespace q27h {
namespace {

#ifndef Q27H_GDN_PARTS
#define Q27H_GDN_PARTS 16  // 8 parts of 16 (one wave per SIMD) measured 616 us vs 574 us at 2048 tokens
#endif
constexpr int kParts = Q27H_GDN_PARTS;  // lanes per column
#ifndef Q27H_GDN_COLS
#define Q27H_GDN_COLS 32
#endif
constexpr int kCols = Q27H_GDN_COLS;    // columns per workgroup
#ifndef Q27H_GDN_GT
#define Q27H_GDN_GT 32
#endif
constexpr int kGT = Q27H_GDN_GT;        // tokens staged per LDS round
#ifndef Q27H_GDN_DEC_COLS
#define Q27H_GDN_DEC_COLS 32
#endif
// Decode (T <= 4 tokens, graph of 64 steps, 48 heads, snapshots): 5.28 against 5.55 us for the prefill form (32
// columns, 32-token staging, plain stores): a 4-token staging round (5.47 us) and nontemporal state-plane stores
// (the planes are next read a whole decode step later). 8 or 16 columns per workgroup (all CUs busy) ran 5.39-5.48 us.
#ifndef Q27H_GDN_SNAP_NT
#define Q27H_GDN_SNAP_NT 1
#endif
constexpr bool kSnapNT = Q27H_GDN_SNAP_NT;  // nontemporal stores of the state planes
constexpr int kDecCols = Q27H_GDN_DEC_COLS;  // columns per workgroup of a decode step (T <= 4, one staging round)

// Sum over the parts of a column (PARTS consecutive lanes): xor butterfly with masks 1, 2, 7 (, 8), which span the
// lane bits of a part index and are all DPP moves (quad_perm, row_half_mirror, row_ror:8). Each step adds a lane
// pair's two values, so every part ends with the bit-identical sum.
template <int PARTS>
__device__ __forceinline__ float parts_sum(float v) {
  v += lane_xor<1>(v);
  v += lane_xor<2>(v);
  v += lane_xor<7>(v);
  if constexpr (PARTS == 16) v += lane_xor<8>(v);
  return v;
}

// One staging round in registers: q / k of GT tokens as float4 pieces (32 per token and vector), v of the
// workgroup's COLS columns, g and beta (the counts round up; pieces past the round are skipped by their guards).
template <int THREADS, int GT, int COLS>
struct Stage {
  static constexpr int NQ = (GT * 32 + THREADS - 1) / THREADS, NV = (GT * COLS + THREADS - 1) / THREADS;
  float4 q[NQ], k[NQ];
  float v[NV];
  float g, b;
};

#ifndef Q27H_GDN_UNROLL
#define Q27H_GDN_UNROLL 32  // full rounds fully unrolled: 509 us for 2048 tokens, 535 us with 1, 544 us with 4
#endif

// SNAP: decode with per-token snapshots (plane t after token t); otherwise only the final state is written. COLS
// columns per workgroup, GT tokens per staging round; the arithmetic of a column does not depend on either.
template <int PARTS, bool SNAP, int COLS = kCols, int GT = kGT>
__global__ void __launch_bounds__(COLS * PARTS) gdn_rec_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                                const float* __restrict__ v, int stride,
                                                                const float* __restrict__ g, const float* __restrict__ beta,
                                                                float* __restrict__ planes, const int* __restrict__ in_plane,
                                                                float* __restrict__ o, int H, int HK, int T, float scale,
                                                                int flip) {
  constexpr int EPL = 128 / PARTS, PAD = EPL + 4, ROW = PARTS * PAD, THREADS = COLS * PARTS;
  // q / k rows padded by 4 floats per part (the parts' float4 reads fall in different banks); two buffers, the
  // next round is loaded while the current one is consumed
  __shared__ __align__(16) float sq[2][GT][ROW];
  __shared__ __align__(16) float sk[2][GT][ROW];
  __shared__ float sv[2][GT][COLS];
  __shared__ float sg[2][GT], sb[2][GT];
  const int h = blockIdx.x, kh = h % HK;
  const int tid = threadIdx.x, p = tid & (PARTS - 1), cl = tid / PARTS, col = blockIdx.y * COLS + cl;
  const size_t plane_sz = (size_t)H * 128 * 128;
  const int pin = *in_plane;
  const size_t soff = ((size_t)h * 128 + col) * 128 + EPL * p;
  float s[EPL];
  {
    const float* src = planes + (size_t)pin * plane_sz + soff;
#pragma unroll
    for (int i = 0; i < EPL; i += 4) {
      const float4 a = ld4(src + i);
      s[i] = a.x; s[i + 1] = a.y; s[i + 2] = a.z; s[i + 3] = a.w;
    }
  }
  using St = Stage<THREADS, GT, COLS>;
  auto load = [&](St& r, int t0) {
    const int nt = min(GT, T - t0);
#pragma unroll
    for (int j = 0; j < St::NQ; j++) {
      const int i = tid + j * THREADS, t = i >> 5, e4 = (i & 31) * 4;
      if (t < nt) {
        r.q[j] = ld4(q + (size_t)(t0 + t) * stride + kh * 128 + e4);
        r.k[j] = ld4(k + (size_t)(t0 + t) * stride + kh * 128 + e4);
      }
    }
#pragma unroll
    for (int j = 0; j < St::NV; j++) {
      const int i = tid + j * THREADS, t = i / COLS, c = i % COLS;
      if (t < nt) r.v[j] = v[(size_t)(t0 + t) * stride + h * 128 + blockIdx.y * COLS + c];
    }
    if (tid < nt) {
      r.g = g[(size_t)(t0 + tid) * H + h];
      r.b = beta[(size_t)(t0 + tid) * H + h];
    }
  };
  auto store = [&](const St& r, int buf, int t0) {
    const int nt = min(GT, T - t0);
#pragma unroll
    for (int j = 0; j < St::NQ; j++) {
      const int i = tid + j * THREADS, t = i >> 5, e4 = (i & 31) * 4, pe = (e4 / EPL) * PAD + e4 % EPL;
      if (t < nt) {
        *(float4*)&sq[buf][t][pe] = r.q[j];
        *(float4*)&sk[buf][t][pe] = r.k[j];
      }
    }
#pragma unroll
    for (int j = 0; j < St::NV; j++) {
      const int i = tid + j * THREADS, t = i / COLS, c = i % COLS;
      if (t < nt) sv[buf][t][c] = r.v[j];
    }
    if (tid < nt) {
      sg[buf][tid] = q27_expf(r.g);
      sb[buf][tid] = r.b;
    }
  };
  const int out_plane = flip ? (pin == 0 ? 1 : 0) : T - 1;
  {
    St r;
    load(r, 0);
    store(r, 0, 0);
  }
  __syncthreads();
  for (int t0 = 0, buf = 0; t0 < T; t0 += GT, buf ^= 1) {
    const int nt = min(GT, T - t0);
    const bool more = t0 + GT < T;
    St r;
    if (more) load(r, t0 + GT);  // in flight during the tokens below
    auto step = [&](int tt) {
      float kr[EPL], qr[EPL];
#pragma unroll
      for (int i = 0; i < EPL; i += 4) {
        const float4 k4 = *(const float4*)&sk[buf][tt][p * PAD + i];
        const float4 q4 = *(const float4*)&sq[buf][tt][p * PAD + i];
        kr[i] = k4.x; kr[i + 1] = k4.y; kr[i + 2] = k4.z; kr[i + 3] = k4.w;
        qr[i] = q4.x; qr[i + 1] = q4.y; qr[i + 2] = q4.z; qr[i + 3] = q4.w;
      }
      float kq[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int i = 0; i < EPL; i++) kq[i & 3] = __builtin_fmaf(s[i], kr[i], kq[i & 3]);
      const float kv = parts_sum<PARTS>((kq[0] + kq[1]) + (kq[2] + kq[3]));
      const float gv = sg[buf][tt];
      const float delta = (sv[buf][tt][cl] - gv * kv) * sb[buf][tt];
      float aq[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int i = 0; i < EPL; i++) {
        s[i] = __builtin_fmaf(kr[i], delta, gv * s[i]);
        aq[i & 3] = __builtin_fmaf(s[i], qr[i], aq[i & 3]);
      }
      const float at = parts_sum<PARTS>((aq[0] + aq[1]) + (aq[2] + aq[3]));
      const int t = t0 + tt;
      if (p == 0) o[((size_t)t * H + h) * 128 + col] = at * scale;
      if (SNAP && t < T - 1) {
        float* W = planes + (size_t)t * plane_sz + soff;
#pragma unroll
        for (int i = 0; i < EPL; i += 4) st4<kSnapNT>(W + i, s[i], s[i + 1], s[i + 2], s[i + 3]);
      }
    };
    if (nt == GT) {
#pragma unroll Q27H_GDN_UNROLL
      for (int tt = 0; tt < GT; tt++) step(tt);
    } else {
      for (int tt = 0; tt < nt; tt++) step(tt);
    }
    if (more) store(r, buf ^ 1, t0 + GT);
    __syncthreads();
  }
  float* W = planes + (size_t)out_plane * plane_sz + soff;
#pragma unroll
  for (int i = 0; i < EPL; i += 4) st4<kSnapNT>(W + i, s[i], s[i + 1], s[i + 2], s[i + 3]);
}

}  // namespace
}  // namespace q27h

using namespace q27h;

// Prefill (flip) runs from kChunkMinT tokens on in the chunked form on matrix cores (gdn_chunk.hip), unless the
// process asked for the sequential, bit-exact kernel. Measured (us, 48 value heads, sequential / chunked): 64 tokens
// 18.7 / 23.1, 96 tokens 26.4 / 27.0, 128 tokens 33.8 / 30.8, 512 tokens 126 / 77, 2048 tokens 491 / 273, 8192
// tokens 2008 / 1078.
constexpr int kChunkMinT = 128;
static std::atomic<int> g_prefill_exact{0};

extern "C" int q27h_gdn_prefill_exact(int on) { return g_prefill_exact.exchange(on ? 1 : 0); }
bool q27h::gdn_prefill_exact_mode() { return g_prefill_exact.load(std::memory_order_relaxed) != 0; }

extern "C" int q27h_gdn_step(const float* q, const float* k, const float* v, int stride, const float* g, const float* beta,
                             float* planes, const int* in_plane, float* o, int H, int HK, int T, float scale, int snapshots,
                             q27h_stream_t s, int flip) {
  if (H <= 0 || HK <= 0 || T < 0 || stride < 128 || stride % 4) return fail(Q27H_ERR_SHAPE, "gdn_step: bad shape");
  if (!flip && T > 4) return fail(Q27H_ERR_SHAPE, "gdn_step: T must be <= 4 without flip (4 state planes)");
  if (T == 0) return Q27H_OK;
  if (!q || !k || !v || !g || !beta || !planes || !in_plane || !o) return fail(Q27H_ERR_ARG, "gdn_step: null pointer");
  if (!aligned16(q) || !aligned16(k) || !aligned16(planes))
    return fail(Q27H_ERR_ARG, "gdn_step: q, k and planes need 16-byte alignment");
  // the switch is read here, when the launch is enqueued: a graph captured under one setting keeps its path
  if (flip && T >= kChunkMinT && !gdn_prefill_exact_mode() &&
      !gdn_chunk_o_overlaps(q, k, v, stride, g, beta, planes, o, H, HK, T))
    return q27h_gdn_step_chunked(q, k, v, stride, g, beta, planes, in_plane, o, H, HK, T, scale, s);
  if (!flip && snapshots && T > 1)
    hipLaunchKernelGGL((gdn_rec_kernel<kParts, true, kDecCols, 4>), dim3(H, 128 / kDecCols), dim3(kDecCols * kParts), 0,
                       stream_of(s), q, k, v, stride, g, beta, planes, in_plane, o, H, HK, T, scale, 0);
  else if (!flip)
    hipLaunchKernelGGL((gdn_rec_kernel<kParts, false, kDecCols, 4>), dim3(H, 128 / kDecCols), dim3(kDecCols * kParts), 0,
                       stream_of(s), q, k, v, stride, g, beta, planes, in_plane, o, H, HK, T, scale, 0);
  else
    hipLaunchKernelGGL((gdn_rec_kernel<kParts, false>), dim3(H, 128 / kCols), dim3(kCols * kParts), 0, stream_of(s), q, k,
                       v, stride, g, beta, planes, in_plane, o, H, HK, T, scale, flip);
  return check_launch("gdn_step");
}
