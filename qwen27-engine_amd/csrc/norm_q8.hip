// Row kernels that end in the q8_1 activation quantization: rmsnorm_q8, sum_norm_q8 / sum_norm_rows /
// add_norm_rows (residual add + RMSNorm), quantize_q8_1, swiglu_q8, gated_rmsnorm_q8, and the unfused twins
// rmsnorm / add / swiglu / gated_rmsnorm that the fused == unfused identity is checked against.
//
// Row engine (n = 5120): one 256-thread workgroup (4 waves) per row. Thread t loads five float4, one per
// 1024-value slice k = 0..4, at the same offset u0 inside each slice (the 32-value block layout of q27h_device.h:
// u0 = 32 (t / 8) + 4 quad_of_lane(t % 8)), so it holds the values of the reference's 1024-thread layout
// (src/ops.cu:110-121: thread u holds u + k*1024) for the four virtual threads u = u0 .. u0+3. The per-virtual-thread partial sums
// of squares, the 32-lane butterflies and the 32-way cross-warp butterfly are then formed from exactly the
// same operands as the reference (q27h_device.h), while every global access is a 16-byte load or store and a
// wave moves 1 KiB per instruction.
#include "q27h_device.h"
#include "q27h_internal.h"

namespace q27h {
namespace {

// ---------------------------------------------------------------- row engine
enum RowMode { kPlain = 0, kAddPartial = 1, kAddBf16Recv = 2, kAddQ8Wire = 3 };
#ifndef Q27H_ROW_NT
#define Q27H_ROW_NT 0
#endif
// Nontemporal stores per kernel (measured in the prefill pass)
#ifndef Q27H_NT_ROW
#define Q27H_NT_ROW 1
#endif
#ifndef Q27H_NT_SWIGLU
#define Q27H_NT_SWIGLU 0
#endif
#ifndef Q27H_NT_QUANT
#define Q27H_NT_QUANT 0
#endif
#ifndef Q27H_NT_GATED
#define Q27H_NT_GATED 0
#endif
#ifndef Q27H_GATED_G
#define Q27H_GATED_G 1  // the prefill pass (2048 tokens, 48 launches): 9.824 ms against 9.892 ms with 2 (three A/B runs on one box)
#endif
constexpr int kGatedG = Q27H_GATED_G;
constexpr int kLatencyRows = 64;  // row launches up to this many rows take the latency-bound kernel variants  // groups of 8 heads per workgroup in gated_rmsnorm_q8
constexpr bool kRowNT = Q27H_NT_ROW, kSwigluNT = Q27H_NT_SWIGLU, kQuantNT = Q27H_NT_QUANT, kGatedNT = Q27H_NT_GATED;
// Q27H_ROW_NT: 0 plain loads, 1 nontemporal loads in every row kernel, 2 nontemporal loads in the prefill-sized
// (non-EXACT) residual-add kernels only
template <bool NTL>
__device__ __forceinline__ float4 ld4_row(const float* p) {
  if constexpr (NTL) return ld4_nt(p);
  else return ld4(p);
}

// MODE kAddQ8Wire: x += dequant(own) + dequant(recv), two q8 wire rows (wown, wrecv: n int8 values, then n / qb fp16
// scales per row; qb = 1 << qb_shift values per scale).
template <int MODE, bool EXACT, bool NTL>
__global__ void __launch_bounds__(256) row_norm_q8_kernel(float* __restrict__ x, const float* __restrict__ partial,
                                                          const uint16_t* __restrict__ recv, const float* __restrict__ w,
                                                          float eps, float* __restrict__ h, int8_t* __restrict__ xq,
                                                          float* __restrict__ xd, float* __restrict__ xs,
                                                          const uint8_t* __restrict__ wown, const uint8_t* __restrict__ wrecv,
                                                          int qb_shift) {
  __shared__ float red[32];
  args_now(x, partial, recv, w, eps, h, xq, xd, xs, wown, wrecv, qb_shift);
  const int t = threadIdx.x;
  const size_t row = blockIdx.x;
  const int off = 32 * (t >> 3) + block_offset(t);  // this thread's 4 values in each 1024-value slice
  const size_t rb = row * kRowN;  // row-relative indices below: 32-bit address arithmetic
  float* const xr = x + rb;
  const float* const pr = partial + rb;
  const uint16_t* const rr = recv + rb;
  // every load of the row first (x, the added operands, w), one memory round trip
  float v[5][4];
  float4 wv[5];
  constexpr int NP = MODE == kAddPartial || MODE == kAddBf16Recv ? 5 : 1;
  constexpr int NR = MODE == kAddBf16Recv ? 5 : 1, NQ = MODE == kAddQ8Wire ? 5 : 1;
  float4 pv4[NP];
  uint2 rv2[NR];
  uint32_t oq[NQ], rq[NQ];
  uint16_t odb[NQ], rdb[NQ];
#pragma unroll
  for (int k = 0; k < 5; k++) {
    const float4 a = ld4_row<NTL>(xr + off + k * 1024);
    v[k][0] = a.x; v[k][1] = a.y; v[k][2] = a.z; v[k][3] = a.w;
  }
  if constexpr (MODE == kAddPartial || MODE == kAddBf16Recv) {
#pragma unroll
    for (int k = 0; k < 5; k++) pv4[k] = ld4_row<NTL>(pr + off + k * 1024);
  }
  if constexpr (MODE == kAddBf16Recv) {
#pragma unroll
    for (int k = 0; k < 5; k++) rv2[k] = *(const uint2*)(rr + off + k * 1024);
  }
  if constexpr (MODE == kAddQ8Wire) {
    const size_t rb = kRowN + ((size_t)2 * kRowN >> qb_shift);
    const uint8_t* ow = wown + row * rb;
    const uint8_t* rw = wrecv + row * rb;
#pragma unroll
    for (int k = 0; k < 5; k++) {
      const int i = off + k * 1024;
      oq[k] = *(const uint32_t*)(ow + i);
      rq[k] = *(const uint32_t*)(rw + i);
      odb[k] = *(const uint16_t*)(ow + kRowN + 2 * (i >> qb_shift));
      rdb[k] = *(const uint16_t*)(rw + kRowN + 2 * (i >> qb_shift));
    }
  }
#pragma unroll
  for (int k = 0; k < 5; k++) wv[k] = ld4(w + off + k * 1024);
  loads_issued();
  if constexpr (MODE == kAddQ8Wire) {
    // x[i] + (d_own q_own + d_recv q_recv): both products are exact (fp16 x int8), the sum rounds once
#pragma unroll
    for (int k = 0; k < 5; k++) {
      const float od = h2f_bits(odb[k]), rd = h2f_bits(rdb[k]);
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const float a = od * (float)(int8_t)(oq[k] >> (8 * c)), b = rd * (float)(int8_t)(rq[k] >> (8 * c));
        v[k][c] = v[k][c] + (a + b);
      }
      st4<kRowNT>(xr + off + k * 1024, v[k][0], v[k][1], v[k][2], v[k][3]);
    }
  } else if constexpr (MODE != kPlain) {
#pragma unroll
    for (int k = 0; k < 5; k++) {
      const float pv[4] = {pv4[k].x, pv4[k].y, pv4[k].z, pv4[k].w};
      if constexpr (MODE == kAddPartial) {
#pragma unroll
        for (int c = 0; c < 4; c++) v[k][c] = v[k][c] + pv[c];
      } else {
        const uint2 rb = rv2[k];
        const float rv[4] = {bf16_to_f((uint16_t)(rb.x & 0xffff)), bf16_to_f((uint16_t)(rb.x >> 16)),
                             bf16_to_f((uint16_t)(rb.y & 0xffff)), bf16_to_f((uint16_t)(rb.y >> 16))};
#pragma unroll
        for (int c = 0; c < 4; c++) v[k][c] = v[k][c] + (bf16_round(pv[c]) + rv[c]);
      }
      st4<kRowNT>(xr + off + k * 1024, v[k][0], v[k][1], v[k][2], v[k][3]);
    }
  }
  // per virtual thread: t = 0; t += v[k]^2 for k = 0..4 (src/ops.cu:96-98)
  float s[4];
#pragma unroll
  for (int c = 0; c < 4; c++) {
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < 5; k++) acc += v[k][c] * v[k][c];
    s[c] = acc;
  }
  const float wsum = vwarp_sum4(s);
  if ((t & 7) == 0) red[t >> 3] = wsum;
  __syncthreads();
  const float tot = red32_sum(red);
  const float scale = 1.0f / __builtin_sqrtf(tot / (float)kRowN + eps);
  float y[5][4];
#pragma unroll
  for (int k = 0; k < 5; k++) {
    const float ww[4] = {wv[k].x, wv[k].y, wv[k].z, wv[k].w};
#pragma unroll
    for (int c = 0; c < 4; c++) y[k][c] = scale * v[k][c] * ww[c];
  }
  if (h) {
#pragma unroll
    for (int k = 0; k < 5; k++) st4<kRowNT>(h + rb + off + k * 1024, y[k][0], y[k][1], y[k][2], y[k][3]);
  }
  q8_1_store_n<kRowNT, 5, EXACT>(y, xq + rb, xd + rb / 32, xs ? xs + rb / 16 : nullptr, off, 1024);
}

// ---------------------------------------------------------------- flat q8_1 producers
// A 256-thread workgroup covers U * 1024 consecutive values; in each 1024-value chunk thread t handles the 4
// values at 32 (t / 8) + 4 quad_of_lane(t % 8) (n % 32 == 0, so a q8 block is the 8 lanes of one group). All loads of a thread are
// issued before any arithmetic so U * 16 (quantize) or U * 32 (swiglu) bytes per lane are in flight.
// Chunks per workgroup, measured in the prefill pass (2048 tokens; two A/B runs on one box): swiglu 1 (9.972 ms
// against 10.010 ms with 2), quantize 2 (10.040 ms with 1).
#ifndef Q27H_FLAT_U
#define Q27H_FLAT_U 1
#endif
#ifndef Q27H_QUANT_U
#define Q27H_QUANT_U 2
#endif
constexpr int kSwigluU = Q27H_FLAT_U, kQuantU = Q27H_QUANT_U;

template <bool SWIGLU, int kFlatU, bool NT, bool EXACT>
__global__ void __launch_bounds__(256) flat_q8_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                      int8_t* __restrict__ xq, float* __restrict__ xd,
                                                      float* __restrict__ xs, size_t n) {
  const size_t wb = (size_t)blockIdx.x * (kFlatU * 1024);  // this workgroup's first value
  const int off = 32 * (threadIdx.x >> 3) + block_offset(threadIdx.x);
  const size_t base = wb + off;
  int8_t* const xq_w = xq + wb;
  float* const xd_w = xd + wb / 32;
  float* const xs_w = xs ? xs + wb / 16 : nullptr;
  float4 a[kFlatU], b[kFlatU];
  int kn = 0;  // chunks of this lane inside n (uniform per 8-lane group: n % 32 == 0)
#pragma unroll
  for (int c = 0; c < kFlatU; c++) {
    const size_t i0 = base + (size_t)c * 1024;
    a[c] = b[c] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (i0 < n) {
      kn = c + 1;
      a[c] = ld4_nt(g + i0);
      if constexpr (SWIGLU) b[c] = ld4_nt(u + i0);
    }
  }
  bool ok = true;  // every silu argument in the fast range (silu_fast_ok)
  float y[kFlatU][4];
#pragma unroll
  for (int c = 0; c < kFlatU; c++) {
    y[c][0] = a[c].x; y[c][1] = a[c].y; y[c][2] = a[c].z; y[c][3] = a[c].w;
    if constexpr (SWIGLU) {
      const float ub[4] = {b[c].x, b[c].y, b[c].z, b[c].w};
#pragma unroll
      for (int k = 0; k < 4; k++) {
        ok &= c >= kn || silu_fast_ok(y[c][k]);
        y[c][k] = silu_fast(y[c][k]) * ub[k];
      }
    }
  }
  q8_1_store_n<NT, kFlatU, EXACT>(y, xq_w, xd_w, xs_w, off, 1024, kn);
  // A wave with a silu argument outside the fast range (practically never) recomputes its values with the general
  // silu and stores them again; in-range values are unchanged.
  if constexpr (SWIGLU) {
    if (__builtin_expect(__any(!ok), 0)) {
#pragma unroll
      for (int c = 0; c < kFlatU; c++) {
        const float gv[4] = {a[c].x, a[c].y, a[c].z, a[c].w}, ub[4] = {b[c].x, b[c].y, b[c].z, b[c].w};
#pragma unroll
        for (int k = 0; k < 4; k++) y[c][k] = q27_silu(gv[k]) * ub[k];
      }
      q8_1_store_n<NT, kFlatU, EXACT>(y, xq_w, xd_w, xs_w, off, 1024, kn);
    }
  }
}

// ---------------------------------------------------------------- gated RMSNorm -> q8_1 (heads of 128)
// 32 lanes per head in the 32-value block layout (4 groups of 8 lanes); each 32-lane half handles kGatedH heads (loads
// of all of them issued first), a 256-thread workgroup 8 * kGatedH heads. The reference's 128-thread block_sum
// (4 warps) becomes: per virtual warp (8 lanes) vwarp_sum4, then the second stage over the 4 warp sums with
// zeros in lanes 4..31, i.e. (w0 + w2) + (w1 + w3) = lane xor 16, then lane xor 8.
// silu(z) is evaluated on the fast range (silu_fast) without a branch, so it overlaps the norm's lane exchanges. A
// wave with any z outside that range (zeros, subnormals, |z| > 60, inf, NaN; practically never) recomputes its
// heads afterwards with the general silu and stores them again: the same addresses, the later store wins, and
// the values of in-range lanes are unchanged.
template <bool NT, int G, bool EXACT>
__global__ void __launch_bounds__(256) gated_rmsnorm_q8_kernel(const float* __restrict__ o, const float* __restrict__ w,
                                                               const float* __restrict__ z, int8_t* __restrict__ xq,
                                                               float* __restrict__ xd, float eps, float* __restrict__ xs,
                                                               int heads) {
  // G groups of 8 heads per workgroup, all of their o / z loads issued before any head is processed; head g of this
  // 32-lane half is head0 + 8 g, so its values sit 1024 after those of head g - 1
  const int p = threadIdx.x & 31;
  const int off = 32 * (p >> 3) + block_offset(p);
  const int head0 = blockIdx.x * G * 8 + (threadIdx.x >> 5);
  const float4 wv = ld4(w + off);
  const float ww[4] = {wv.x, wv.y, wv.z, wv.w};
  float4 zv[G], ov[G];
  int kn = 0;  // heads of this 32-lane half inside `heads`
#pragma unroll
  for (int g = 0; g < G; g++) {
    const int head = head0 + 8 * g;
    zv[g] = ov[g] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (head < heads) {  // uniform per 32-lane half
      kn = g + 1;
      const size_t i0 = (size_t)head * 128 + off;
      zv[g] = ld4_nt(z + i0);  // z first: silu(z) is computed first
      ov[g] = ld4_nt(o + i0);
    }
  }
  float y[G][4], sc[G];
  bool ok = true;
#pragma unroll
  for (int g = 0; g < G; g++) {
    const float v[4] = {ov[g].x, ov[g].y, ov[g].z, ov[g].w};
    const float zz[4] = {zv[g].x, zv[g].y, zv[g].z, zv[g].w};
    float gz[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
      gz[c] = silu_fast(zz[c]);
      ok &= g >= kn || silu_fast_ok(zz[c]);
    }
    float s[4];
#pragma unroll
    for (int c = 0; c < 4; c++) s[c] = v[c] * v[c];
    float tsum = vwarp_sum4(s);
    tsum = tsum + 0.0f;  // the reference adds the zero lanes 4..31 (xor 16, 8, 4 steps); x + 0 == x for x >= +0
    tsum += lane_xor<16>(tsum);
    tsum += lane_xor<8>(tsum);
    sc[g] = 1.0f / __builtin_sqrtf(tsum / 128.0f + eps);
#pragma unroll
    for (int c = 0; c < 4; c++) y[g][c] = (sc[g] * v[c] * ww[c]) * gz[c];
  }
  const size_t wb = (size_t)blockIdx.x * G * 8 * 128;  // this workgroup's first value
  const int i0 = (threadIdx.x >> 5) * 128 + off;
  int8_t* const xq_w = xq + wb;
  float* const xd_w = xd + wb / 32;
  float* const xs_w = xs ? xs + wb / 16 : nullptr;
  q8_1_store_n<NT, G, EXACT>(y, xq_w, xd_w, xs_w, i0, 1024, kn);
  if (__builtin_expect(__any(!ok), 0)) {
#pragma unroll
    for (int g = 0; g < G; g++) {
      const float v[4] = {ov[g].x, ov[g].y, ov[g].z, ov[g].w};
      const float zz[4] = {zv[g].x, zv[g].y, zv[g].z, zv[g].w};
#pragma unroll
      for (int c = 0; c < 4; c++) y[g][c] = (sc[g] * v[c] * ww[c]) * q27_silu(zz[c]);
    }
    q8_1_store_n<NT, G, EXACT>(y, xq_w, xd_w, xs_w, i0, 1024, kn);
  }
}

// ---------------------------------------------------------------- unfused twins (reference structure)
// rmsnorm_kernel (src/ops.cu:57-68): block of B threads per row, thread t sums x[i]^2 for i = t, t + B, ...
__global__ void __launch_bounds__(1024) rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                       float* __restrict__ y, int n, float eps, int ystride) {
  __shared__ float red[32];
  const float* xr = x + (size_t)blockIdx.x * n;
  float* yr = y + (size_t)blockIdx.x * ystride;
  float t = 0.0f;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const float v = xr[i];
    t += v * v;
  }
  t = block_sum_ref(t, red, blockDim.x);
  const float scale = 1.0f / __builtin_sqrtf(t / (float)n + eps);
  for (int i = threadIdx.x; i < n; i += blockDim.x) yr[i] = scale * xr[i] * w[i];
}

__global__ void add_kernel(const float* __restrict__ x, const float* __restrict__ a, float* __restrict__ y, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = x[i] + a[i];
}

__global__ void swiglu_kernel(const float* __restrict__ g, const float* __restrict__ u, float* __restrict__ y, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    const float gi[1] = {g[i]};
    float sg[1];
    q27_silu_n(gi, sg);
    y[i] = sg[0] * u[i];
  }
}

__global__ void set_int_kernel(int* p, int v) { *p = v; }

// gated_rmsnorm_kernel (src/ops.cu:574-585): 128 threads per head of n values.
__global__ void __launch_bounds__(128) gated_rmsnorm_kernel(const float* __restrict__ o, const float* __restrict__ w,
                                                            const float* __restrict__ z, float* __restrict__ y, int n,
                                                            float eps) {
  __shared__ float red[32];
  const size_t off = (size_t)blockIdx.x * n;
  float t = 0.0f;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const float v = o[off + i];
    t += v * v;
  }
  t = block_sum_ref(t, red, blockDim.x);
  const float scale = 1.0f / __builtin_sqrtf(t / (float)n + eps);
  for (int i = threadIdx.x; i < n; i += blockDim.x) y[off + i] = (scale * o[off + i] * w[i]) * q27_silu(z[off + i]);
}

int check_row_args(const char* fn, int n, int rows, const float* x, const float* w, const float* h, const int8_t* xq,
                   const float* xd) {
  if (n != kRowN) return fail(Q27H_ERR_SHAPE, std::string(fn) + ": n must be 5120");
  if (rows < 0) return fail(Q27H_ERR_SHAPE, std::string(fn) + ": rows < 0");
  if (!x || !w || !xq || !xd) return fail(Q27H_ERR_ARG, std::string(fn) + ": null pointer");
  if (!aligned16(x) || !aligned16(w) || (h && !aligned16(h)) || !aligned4(xq))
    return fail(Q27H_ERR_ARG, std::string(fn) + ": x, w, h need 16-byte and xq 4-byte alignment");
  return Q27H_OK;
}

template <int MODE>
int launch_rows(const char* fn, float* x, const float* partial, const uint16_t* recv, const float* w, float eps, float* h,
                int8_t* xq, float* xd, float* xs, int rows, q27h_stream_t s, const uint8_t* wown = nullptr,
                const uint8_t* wrecv = nullptr, int qb_shift = 0) {
  if (rows == 0) return Q27H_OK;
  // Branch-free quotients (q8_quot_exact) at every size: latency-bound launches (a few workgroups per chip) gain the
  // shorter chain, and in the 2048-row prefill pass they measured 9.72 against 9.86 ms per pass with the reciprocal
  // fast path (two A/B runs on one box; the row kernel's waves otherwise often wait on a fallback block). A
  // 1024-thread form with 5 values per lane, the reference's layout, measured slower: 4.0 against 3.3 us per decode
  // node. A persistent form (a grid of 1-4 workgroups per CU, each walking rows with the next row's loads in flight)
  // measured slower at 2048 rows: 30.0-31.7 against 27.6 us for sum_norm_rows. Fewer resident workgroups per CU
  // (dynamic LDS of 32, 40 or 54 KB per workgroup) made no difference to the pass; 80 KB made it 8% slower. The
  // in-place x store right after the loads, before the reduction, is worth 140 us per pass against storing x after
  // it beside the q8_1 output (10.41-10.48 against 10.55-10.61 ms).
  if (Q27H_ROW_NT == 2 && MODE != kPlain && rows > kLatencyRows)
    hipLaunchKernelGGL((row_norm_q8_kernel<MODE, true, true>), dim3(rows), dim3(256), 0, stream_of(s), x, partial, recv,
                       w, eps, h, xq, xd, xs, wown, wrecv, qb_shift);
  else
    hipLaunchKernelGGL((row_norm_q8_kernel<MODE, true, Q27H_ROW_NT == 1>), dim3(rows), dim3(256), 0, stream_of(s), x,
                       partial, recv, w, eps, h, xq, xd, xs, wown, wrecv, qb_shift);
  return check_launch(fn);
}

int launch_flat(const char* fn, bool swiglu, const float* g, const float* u, int8_t* xq, float* xd, float* xs, size_t n,
                q27h_stream_t s) {
  if (n == 0) return Q27H_OK;
  if (!g || !xq || !xd || (swiglu && !u)) return fail(Q27H_ERR_ARG, std::string(fn) + ": null pointer");
  if (!aligned16(g) || (swiglu && !aligned16(u)) || !aligned4(xq))
    return fail(Q27H_ERR_ARG, std::string(fn) + ": inputs need 16-byte and xq 4-byte alignment");
  // a launch of a few workgroups per chip is latency-bound: one 1024-value chunk per workgroup (the shortest chain
  // per lane) and branch-free quotients
  const bool lat = n <= (size_t)kLatencyRows * kRowN;
  const int U = lat ? 1 : swiglu ? kSwigluU : kQuantU;
  const dim3 grid((unsigned)((n + U * 1024 - 1) / (U * 1024))), block(256);
  if (swiglu && lat)
    hipLaunchKernelGGL((flat_q8_kernel<true, 1, kSwigluNT, true>), grid, block, 0, stream_of(s), g, u, xq, xd, xs, n);
  else if (swiglu)
    hipLaunchKernelGGL((flat_q8_kernel<true, kSwigluU, kSwigluNT, false>), grid, block, 0, stream_of(s), g, u, xq, xd, xs, n);
  else if (lat)
    hipLaunchKernelGGL((flat_q8_kernel<false, 1, kQuantNT, true>), grid, block, 0, stream_of(s), g, u, xq, xd, xs, n);
  else
    hipLaunchKernelGGL((flat_q8_kernel<false, kQuantU, kQuantNT, false>), grid, block, 0, stream_of(s), g, u, xq, xd, xs, n);
  return check_launch(fn);
}

}  // namespace
}  // namespace q27h

using namespace q27h;

extern "C" int q27h_rmsnorm_q8(const float* x, const float* w, float* h, int8_t* xq, float* xd, int n, int rows, float eps,
                               q27h_stream_t s, float* xs) {
  if (int e = check_row_args("rmsnorm_q8", n, rows, x, w, h, xq, xd)) return e;
  return launch_rows<kPlain>("rmsnorm_q8", const_cast<float*>(x), nullptr, nullptr, w, eps, h, xq, xd, xs, rows, s);
}

extern "C" int q27h_sum_norm_q8(float* x, const float* partial, int n, int rows, const void* ar, const float* w, float eps,
                                float* h, int8_t* xq, float* xd, q27h_stream_t s, const void* pf, size_t pf_bytes) {
  (void)pf;
  (void)pf_bytes;
  if (ar) return fail(Q27H_ERR_UNSUPPORTED, "sum_norm_q8: the cross-card exchange (ar != null) is not part of this build");
  if (int e = check_row_args("sum_norm_q8", n, rows, x, w, h, xq, xd)) return e;
  if (!partial || !aligned16(partial)) return fail(Q27H_ERR_ARG, "sum_norm_q8: partial null or misaligned");
  return launch_rows<kAddPartial>("sum_norm_q8", x, partial, nullptr, w, eps, h, xq, xd, nullptr, rows, s);
}

extern "C" int q27h_sum_norm_rows(float* x, const float* partial, int n, int M, const void* ex, const float* w, float eps,
                                  float* h, int8_t* xq, float* xd, float* xs, q27h_stream_t s) {
  if (ex) return fail(Q27H_ERR_UNSUPPORTED, "sum_norm_rows: the cross-card exchange (ex != null) is not part of this build");
  if (int e = check_row_args("sum_norm_rows", n, M, x, w, h, xq, xd)) return e;
  if (!partial || !aligned16(partial)) return fail(Q27H_ERR_ARG, "sum_norm_rows: partial null or misaligned");
  return launch_rows<kAddPartial>("sum_norm_rows", x, partial, nullptr, w, eps, h, xq, xd, xs, M, s);
}

extern "C" int q27h_add_norm_rows(float* x, const float* partial, const uint16_t* recv, int n, int M, const float* w,
                                  float eps, float* h, int8_t* xq, float* xd, float* xs, q27h_stream_t s) {
  if (int e = check_row_args("add_norm_rows", n, M, x, w, h, xq, xd)) return e;
  if (!partial || !aligned16(partial)) return fail(Q27H_ERR_ARG, "add_norm_rows: partial null or misaligned");
  if (recv) {
    if (((uintptr_t)recv & 7u) != 0) return fail(Q27H_ERR_ARG, "add_norm_rows: recv needs 8-byte alignment");
    return launch_rows<kAddBf16Recv>("add_norm_rows", x, partial, recv, w, eps, h, xq, xd, xs, M, s);
  }
  return launch_rows<kAddPartial>("add_norm_rows", x, partial, nullptr, w, eps, h, xq, xd, xs, M, s);
}

extern "C" int q27h_add_norm_rows_q8(float* x, const uint8_t* own, const uint8_t* recv, int n, int M, const float* w,
                                     float eps, float* h, int8_t* xq, float* xd, float* xs, int qb, q27h_stream_t s) {
  if (qb != 16 && qb != 32) return fail(Q27H_ERR_SHAPE, "add_norm_rows_q8: qb must be 16 or 32 (the q8 wires)");
  if (int e = check_row_args("add_norm_rows_q8", n, M, x, w, h, xq, xd)) return e;
  if (M > 0 && (!own || !recv)) return fail(Q27H_ERR_ARG, "add_norm_rows_q8: null wire");
  if (!aligned16(own) || !aligned16(recv)) return fail(Q27H_ERR_ARG, "add_norm_rows_q8: wires need 16-byte alignment");
  return launch_rows<kAddQ8Wire>("add_norm_rows_q8", x, nullptr, nullptr, w, eps, h, xq, xd, xs, M, s, own, recv,
                                 qb == 16 ? 4 : 5);
}

extern "C" int q27h_quantize_q8_1(const float* x, int8_t* xq, float* xd, int K, int ncols, q27h_stream_t s, float* xs) {
  if (K <= 0 || K % 32 || ncols < 0) return fail(Q27H_ERR_SHAPE, "quantize_q8_1: K must be a positive multiple of 32");
  return launch_flat("quantize_q8_1", false, x, nullptr, xq, xd, xs, (size_t)K * (size_t)ncols, s);
}

extern "C" int q27h_swiglu_q8(const float* g, const float* u, int8_t* xq, float* xd, int n, q27h_stream_t s, float* xs) {
  if (n < 0 || n % 32) return fail(Q27H_ERR_SHAPE, "swiglu_q8: n % 32");
  return launch_flat("swiglu_q8", true, g, u, xq, xd, xs, (size_t)n, s);
}

extern "C" int q27h_gated_rmsnorm_q8(const float* o, const float* w, const float* z, int8_t* xq, float* xd, int heads,
                                     float eps, q27h_stream_t s, float* xs) {
  if (heads < 0) return fail(Q27H_ERR_SHAPE, "gated_rmsnorm_q8: heads < 0");
  if (heads == 0) return Q27H_OK;
  if (!o || !w || !z || !xq || !xd) return fail(Q27H_ERR_ARG, "gated_rmsnorm_q8: null pointer");
  if (!aligned16(o) || !aligned16(w) || !aligned16(z) || !aligned4(xq))
    return fail(Q27H_ERR_ARG, "gated_rmsnorm_q8: o, w, z need 16-byte and xq 4-byte alignment");
  if (heads <= 8 * kLatencyRows)  // decode: a few workgroups per chip, latency-bound; one head per 32-lane half
    hipLaunchKernelGGL((gated_rmsnorm_q8_kernel<kGatedNT, 1, true>), dim3((heads + 7) / 8), dim3(256), 0, stream_of(s), o, w, z,
                       xq, xd, eps, xs, heads);
  else
    hipLaunchKernelGGL((gated_rmsnorm_q8_kernel<kGatedNT, kGatedG, false>), dim3((heads + 8 * kGatedG - 1) / (8 * kGatedG)),
                       dim3(256), 0, stream_of(s), o, w, z, xq, xd, eps, xs, heads);
  return check_launch("gated_rmsnorm_q8");
}

extern "C" int q27h_rmsnorm(const float* x, const float* w, float* y, int n, int rows, float eps, q27h_stream_t s,
                            int ystride) {
  if (n <= 0 || rows < 0) return fail(Q27H_ERR_SHAPE, "rmsnorm: bad shape");
  if (rows == 0) return Q27H_OK;
  if (!x || !w || !y) return fail(Q27H_ERR_ARG, "rmsnorm: null pointer");
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(n >= 1024 ? 1024 : 256), 0, stream_of(s), x, w, y, n, eps,
                     ystride ? ystride : n);
  return check_launch("rmsnorm");
}

extern "C" int q27h_add(const float* x, const float* a, float* y, int n, q27h_stream_t s) {
  if (n < 0) return fail(Q27H_ERR_SHAPE, "add: n < 0");
  if (n == 0) return Q27H_OK;
  hipLaunchKernelGGL(add_kernel, dim3((n + 255) / 256), dim3(256), 0, stream_of(s), x, a, y, n);
  return check_launch("add");
}

extern "C" int q27h_swiglu(const float* g, const float* u, float* y, int n, q27h_stream_t s) {
  if (n < 0) return fail(Q27H_ERR_SHAPE, "swiglu: n < 0");
  if (n == 0) return Q27H_OK;
  hipLaunchKernelGGL(swiglu_kernel, dim3((n + 255) / 256), dim3(256), 0, stream_of(s), g, u, y, n);
  return check_launch("swiglu");
}

extern "C" int q27h_set_int(int* p, int v, q27h_stream_t s) {
  if (!p) return fail(Q27H_ERR_ARG, "set_int: null pointer");
  hipLaunchKernelGGL(set_int_kernel, dim3(1), dim3(1), 0, stream_of(s), p, v);
  return check_launch("set_int");
}

extern "C" int q27h_gated_rmsnorm(const float* o, const float* w, const float* z, float* y, int n, int heads, float eps,
                                  q27h_stream_t s) {
  if (n <= 0 || heads < 0) return fail(Q27H_ERR_SHAPE, "gated_rmsnorm: bad shape");
  if (heads == 0) return Q27H_OK;
  hipLaunchKernelGGL(gated_rmsnorm_kernel, dim3(heads), dim3(128), 0, stream_of(s), o, w, z, y, n, eps);
  return check_launch("gated_rmsnorm");
}
