// Gated-DeltaNet recurrence, prefill (flip) mode, in the chunked form on fp32 matrix cores (gdn_step with flip,
// src/ops.h:40-45, src/ops.cu:449-572). Same inputs, outputs and plane semantics as the sequential kernel
// (gdn_rec.hip); the additions happen in another order, so the results agree with it to fp32 rounding, not bit for bit.
//
// Per value head h and chunk of C = 16 tokens (G_c = g_0 + ... + g_c, gamma_c = e^G_c, D_cs = e^(G_c - G_s)):
//   A     = strictly lower part of beta_c D_cs (k_c . k_s)            (C x C)
//   Tinv  = (I + A)^-1 = (I - A)(I + A^2)(I + A^4)(I + A^8)          (A^16 = 0)
//   M     = lower part, diagonal included, of D_cs (q_c . k_s)
//   Delta = Tinv (beta (V - gamma (K S)))                              (C x cols: the tokens' delta vectors)
//   O     = scale (gamma (Q S) + M Delta)
//   S    <- gamma_15 S + sum_s D_15,s k_s Delta_s^T
// which unrolls the per-token rule  delta = (v - e^g S^T k) beta,  S <- e^g S + k delta^T,  o = scale S^T q  over the
// chunk (the sequential kernel's comment gives the per-token form).
//
// Two launches. gdn_chunk_prep_kernel (one wave per key head and chunk, all chunks in parallel) forms Tinv and M,
// which do not depend on the state, and parks them where the second launch finds them: for a full chunk in the
// chunk's own rows of o (one 16 x 32 copy per 32-column group of the head, [t][j] = Tinv[t][j] for j < 16, M[t][j - 16]
// otherwise), which the recurrence overwrites only with that group's own outputs after reading them; for a last,
// partial chunk in the output state plane (keys 0..15 of the group's 32 columns), written only at the very end.
// gdn_chunk_kernel then walks the chunks of one value head and 32 value columns (grid H x 4, 512 threads): wave w
// holds the state rows 32 (w & 3) .. + 31 of the columns 16 (w >> 2) .. + 15 as two 16 x 16 accumulator tiles of
// v_mfma_f32_16x16x4_f32 (lane l: rows 4 (l / 16) + i, column l % 16). K S and Q S are split over the 4 row groups of
// a column half (their operand steps read keys in the state tile's own row order, so the state never leaves its
// accumulators); Delta and O are formed by one wave per column half, with the 16 x 16 right-hand side turned into
// MFMA operands by lane swaps; the update is an MFMA into the state tiles. A chunk's rows (k, q, v, g, beta, Tinv, M)
// are loaded kNB - 1 = three chunks ahead into one of four LDS buffers.
#include "q27h_device.h"
#include "q27h_internal.h"

namespace q27h {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
constexpr int kC = 16;     // tokens per chunk
constexpr int kNC = 32;    // value columns per workgroup of the recurrence
constexpr int kKP = 132;   // padded LDS row of a chunk's k / q (floats)
constexpr int kMP = 17;    // padded LDS row of the 16 x 16 matrices
// row buffers of the recurrence: rows are loaded kNB - 1 chunks ahead (3, 4 or 5 buffers measured the same:
// 282-290 us per 2048-token layer)
constexpr int kNB = 4;

__device__ __forceinline__ v4f mfma4(float a, float b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// A 16 x 16 tile in the accumulator layout (lane l = (g, c), g = l / 16: rows 4 g .. 4 g + 3 of column c) to the
// MFMA B-operand layout (step m of lane (g, c): row 4 m + g of column c), i.e. a 4 x 4 transpose of (lane row,
// element) per column: v_permlane32_swap exchanges bit 1 of the two indices, v_permlane16_swap bit 0.
__device__ __forceinline__ v4f tile_to_operand(v4f x) {
  int e[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const float f = x[i];  // through a scalar: __builtin_bit_cast of a vector element reads element 0 with this clang
    e[i] = __builtin_bit_cast(int, f);
  }
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const auto p = __builtin_amdgcn_permlane32_swap(e[i], e[i + 2], false, false);
    e[i] = (int)p[0];
    e[i + 2] = (int)p[1];
  }
#pragma unroll
  for (int i = 0; i < 4; i += 2) {
    const auto p = __builtin_amdgcn_permlane16_swap(e[i], e[i + 1], false, false);
    e[i] = (int)p[0];
    e[i + 1] = (int)p[1];
  }
  v4f y;
#pragma unroll
  for (int i = 0; i < 4; i++) y[i] = __builtin_bit_cast(float, e[i]);
  return y;
}

// X Y^T of two 16 x 128 row blocks in LDS over all 128 columns, by one wave, in the accumulator layout. MFMA step m
// takes column 16 (m / 4) + 4 (l / 16) + m % 4 on both operands (16-byte reads), four accumulators keep the steps
// independent.
__device__ __forceinline__ v4f gram16(const float (*X)[kKP], const float (*Y)[kKP], int r, int kq) {
  v4f acc[4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const float4 x4 = *(const float4*)&X[r][16 * j + 4 * kq];
    const float4 y4 = *(const float4*)&Y[r][16 * j + 4 * kq];
    acc[0] = mfma4(x4.x, y4.x, acc[0]);
    acc[1] = mfma4(x4.y, y4.y, acc[1]);
    acc[2] = mfma4(x4.z, y4.z, acc[2]);
    acc[3] = mfma4(x4.w, y4.w, acc[3]);
  }
  return (acc[0] + acc[1]) + (acc[2] + acc[3]);
}

// G_t = g_0 + ... + g_t (token order) on lane t < 16 (lanes >= 16: the sum of all 16), g[16] in LDS, 16-byte aligned
__device__ __forceinline__ float prefix16(const float* g, int l) {
  float gv[kC];
#pragma unroll
  for (int j = 0; j < kC; j += 4) {  // read unconditionally (a select per term, not a masked read per term)
    const float4 g4 = *(const float4*)&g[j];
    gv[j] = g4.x; gv[j + 1] = g4.y; gv[j + 2] = g4.z; gv[j + 3] = g4.w;
  }
  float G = 0.0f;
#pragma unroll
  for (int j = 0; j < kC; j++) G += j <= l ? gv[j] : 0.0f;
  return G;
}

// (I + B)^-1 = (I + B)(I + B^2)(I + B^4)(I + B^8) for strictly lower B [16][kMP] in LDS, by one wave, in registers:
// every product Z = X Y is formed with its transpose (Z^T = Y^T X^T, a second MFMA chain), both turned into B-operand
// tiles, so the next product reads both operands from registers (the A operand of X is the B operand of X^T).
// Result in the accumulator layout.
__device__ __forceinline__ v4f unit_lower_inverse(const float (*B)[kMP], int r, int kq) {
  v4f bB, bBt;  // B-operand tiles of B and B^T
#pragma unroll
  for (int m = 0; m < 4; m++) {
    bB[m] = B[4 * m + kq][r];
    bBt[m] = B[r][4 * m + kq];
  }
  auto addI = [&](v4f x) {  // (I + X) in the B-operand layout: step m holds row 4 m + kq of column r
#pragma unroll
    for (int m = 0; m < 4; m++) x[m] += (4 * m + kq == r) ? 1.0f : 0.0f;
    return x;
  };
  auto mm = [&](v4f xt, v4f y) {  // Z = X Y from the B-operand tiles of X^T and Y; Z in the accumulator layout
    v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < 4; m++) acc = mfma4(xt[m], y[m], acc);
    return acc;
  };
  const v4f b2 = tile_to_operand(mm(bBt, bB)), b2t = tile_to_operand(mm(bB, bBt));
  const v4f b4 = tile_to_operand(mm(b2t, b2)), b4t = tile_to_operand(mm(b2, b2t));
  const v4f p1t = tile_to_operand(mm(addI(b2), addI(bBt)));  // ((I + B)(I + B^2))^T = (I + B^2^T)(I + B^T)
  const v4f b8 = tile_to_operand(mm(b4t, b4));
  const v4f p2t = tile_to_operand(mm(addI(b4), p1t));  // ((I + B)(I + B^2)(I + B^4))^T
  return mm(p2t, addI(b8));
}

// ---------------------------------------------------------------- prep: Tinv and M of every chunk
// One wave per (key head, chunk): K K^T and Q K^T once, then Tinv and M of every value head on that key head (their
// g and beta differ).
__global__ void __launch_bounds__(64) gdn_chunk_prep_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                            int stride, const float* __restrict__ g,
                                                            const float* __restrict__ beta, float* __restrict__ planes,
                                                            const int* __restrict__ in_plane, float* __restrict__ o,
                                                            int H, int HK, int T) {
  __shared__ __align__(16) float sK[kC][kKP];
  __shared__ __align__(16) float sQ[kC][kKP];
  __shared__ __align__(16) float sg[kC];
  __shared__ float sb[kC];
  __shared__ float sB[kC][kMP];
  const int kh = blockIdx.x, c = blockIdx.y;
  const int c0 = c * kC, n = min(kC, T - c0);
  const int l = threadIdx.x, r = l & 15, kq = l >> 4;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const int e = l + 64 * j, t = e >> 5, e4 = (e & 31) * 4;
    float4 kv4 = make_float4(0.f, 0.f, 0.f, 0.f), qv4 = kv4;
    if (t < n) {
      kv4 = ld4(k + (size_t)(c0 + t) * stride + kh * 128 + e4);
      qv4 = ld4(q + (size_t)(c0 + t) * stride + kh * 128 + e4);
    }
    *(float4*)&sK[t][e4] = kv4;
    *(float4*)&sQ[t][e4] = qv4;
  }
  __syncthreads();
  const v4f kk = gram16(sK, sK, r, kq), qk = gram16(sQ, sK, r, kq);
  const size_t plane_sz = (size_t)H * 128 * 128;
  const int pout = *in_plane == 0 ? 1 : 0;
  for (int h = kh; h < H; h += HK) {
    if (l < kC) {
      sg[l] = l < n ? g[(size_t)(c0 + l) * H + h] : 0.0f;
      sb[l] = l < n ? beta[(size_t)(c0 + l) * H + h] : 0.0f;
    }
    __syncthreads();
    const float Gt = prefix16(sg, l);
    const float Gs = __shfl(Gt, r, 64);
    v4f mt;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int cc = 4 * kq + i;
      const float Gc = __shfl(Gt, cc, 64);  // every lane takes part (a lane exchange reads from active lanes only)
      const float d = r <= cc ? q27_expf(Gc - Gs) : 0.0f;
      sB[cc][r] = r < cc ? -((sb[cc] * d) * kk[i]) : 0.0f;
      mt[i] = r <= cc ? d * qk[i] : 0.0f;
    }
    __syncthreads();
    const v4f ti = unit_lower_inverse(sB, r, kq);
#pragma unroll
    for (int cg = 0; cg < 128 / kNC; cg++) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int t = 4 * kq + i;
        if (n == kC) {
          float* dst = o + ((size_t)(c0 + t) * H + h) * 128 + kNC * cg;
          dst[r] = ti[i];
          dst[16 + r] = mt[i];
        } else {
          float* dst = planes + (size_t)pout * plane_sz + ((size_t)h * 128 + kNC * cg) * 128 + t;
          dst[(size_t)r * 128] = ti[i];
          dst[(size_t)(16 + r) * 128] = mt[i];
        }
      }
    }
    __syncthreads();  // sg, sb and sB are refilled for the next value head
  }
}

// ---------------------------------------------------------------- the recurrence over the chunks
__global__ void __launch_bounds__(512) gdn_chunk_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                        const float* __restrict__ v, int stride,
                                                        const float* __restrict__ g, const float* __restrict__ beta,
                                                        float* __restrict__ planes, const int* __restrict__ in_plane,
                                                        float* __restrict__ o, int H, int HK, int T, float scale) {
  // a chunk's rows, kNB buffers (chunk n in use, the next ones waiting, n + kNB - 1 arriving)
  __shared__ __align__(16) float sKb[kNB][kC][kKP];
  __shared__ __align__(16) float sQb[kNB][kC][kKP];
  __shared__ float sVb[kNB][kC][kNC];
  __shared__ __align__(16) float sgb[kNB][kC];
  __shared__ float sbb[kNB][kC];
  __shared__ float sTb[kNB][kC][kMP], sMb[kNB][kC][kMP];
  __shared__ float sgam[2][kC], sdec[2][kC];    // decays of chunks n and n + 1
  __shared__ __align__(16) v4f part[8][2][64];  // K S, Q S partial tiles
  __shared__ float sDl[2][kC][kMP];             // Delta of the two column halves
  const int h = blockIdx.x, kh = h % HK, cg = blockIdx.y;
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, r = l & 15, kq = l >> 4;
  const int kb = w & 3, cb = w >> 2;
  // Delta / O of column half 0 on wave 0, of half 1 on wave 5 (waves w and w + 4 share a SIMD), decays on wave 2
  const bool dl_wave = w == 0 || w == 5;
  const int col = cg * kNC + cb * 16 + r;  // this lane's value column (state tile column)
  const size_t plane_sz = (size_t)H * 128 * 128;
  const int pin = *in_plane, pout = pin == 0 ? 1 : 0;
  const int nch = (T + kC - 1) / kC;
  v4f S[2];
  {
    const float* src = planes + (size_t)pin * plane_sz + ((size_t)h * 128 + col) * 128 + 32 * kb + 4 * kq;
#pragma unroll
    for (int b = 0; b < 2; b++) {
      const float4 a = ld4(src + 16 * b);
      S[b] = v4f{a.x, a.y, a.z, a.w};
    }
  }
  const int st_t = tid >> 5, st_e4 = (tid & 31) * 4, st_c = tid & 31;
  float4 pk, pq;
  float pv, pt, pg = 0.0f, pb = 0.0f;
  auto fetch = [&](int ch) {  // chunk ch's rows into registers (zeros, and no loads, past T)
    const int c0 = ch * kC, n = min(kC, T - c0);
    pk = make_float4(0.f, 0.f, 0.f, 0.f);
    pq = pk;
    pv = 0.0f;
    pt = 0.0f;
    if (st_t < n) {
      pk = ld4(k + (size_t)(c0 + st_t) * stride + kh * 128 + st_e4);
      pq = ld4(q + (size_t)(c0 + st_t) * stride + kh * 128 + st_e4);
      pv = v[(size_t)(c0 + st_t) * stride + h * 128 + cg * kNC + st_c];
    }
    if (n == kC) pt = o[((size_t)(c0 + st_t) * H + h) * 128 + cg * kNC + st_c];  // Tinv / M, parked in o
    else if (n > 0) pt = planes[(size_t)pout * plane_sz + ((size_t)h * 128 + cg * kNC + st_c) * 128 + st_t];
    if (tid < kC) {
      pg = tid < n ? g[(size_t)(c0 + tid) * H + h] : 0.0f;
      pb = tid < n ? beta[(size_t)(c0 + tid) * H + h] : 0.0f;
    }
  };
  auto stash = [&](int buf) {
    *(float4*)&sKb[buf][st_t][st_e4] = pk;
    *(float4*)&sQb[buf][st_t][st_e4] = pq;
    sVb[buf][st_t][st_c] = pv;
    if (st_c < 16) sTb[buf][st_t][st_c] = pt;
    else sMb[buf][st_t][st_c - 16] = pt;
    if (tid < kC) {
      sgb[buf][tid] = pg;
      sbb[buf][tid] = pb;
    }
  };
  // gamma_t = e^G_t and dec_t = e^(G_15 - G_t) of chunk ch, by one wave
  auto decays = [&](int ch) {
    const float Gt = prefix16(sgb[ch % kNB], l);
    const float G15 = __shfl(Gt, kC - 1, 64);
    if (l < kC) {
      sgam[ch & 1][l] = q27_expf(Gt);
      sdec[ch & 1][l] = q27_expf(G15 - Gt);
    }
  };

  for (int c = 0; c < kNB - 1; c++) {
    fetch(c);
    stash(c);
  }
  __syncthreads();
  if (w == 2) decays(0);
  __syncthreads();

  for (int ch = 0; ch < nch; ch++) {
    const int c0 = ch * kC, n = min(kC, T - c0);
    const int rb = ch % kNB, db = ch & 1;
    // chunk ch + kNB - 1, in flight during this chunk and stored at its end (past the last chunk: no loads, zeros into a
    // buffer no later chunk reads; unconditional, which keeps the compiler's memory-counter waits exact)
    fetch(ch + kNB - 1);
    // ---- X: partial K S, Q S of chunk ch over this wave's 32 state rows
    {
      v4f ks = {0.f, 0.f, 0.f, 0.f}, qs = ks;
#pragma unroll
      for (int b = 0; b < 2; b++) {
        const float4 k4 = *(const float4*)&sKb[rb][r][32 * kb + 16 * b + 4 * kq];
        const float4 q4 = *(const float4*)&sQb[rb][r][32 * kb + 16 * b + 4 * kq];
        const float kr[4] = {k4.x, k4.y, k4.z, k4.w}, qr[4] = {q4.x, q4.y, q4.z, q4.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
          ks = mfma4(kr[i], S[b][i], ks);
          qs = mfma4(qr[i], S[b][i], qs);
        }
      }
      part[w][0][l] = ks;
      part[w][1][l] = qs;
    }
    __syncthreads();
    // ---- Y: Delta = Tinv (beta (V - gamma K S)) and O = gamma Q S + M Delta (one wave per column half);
    //      the decays of chunk ch + 1
    v4f oz;  // this chunk's output tile (the Delta waves), stored at the end of the chunk
    if (dl_wave) {
      v4f ks = part[4 * cb][0][l], qs = part[4 * cb][1][l];
#pragma unroll
      for (int j = 1; j < 4; j++) {
        ks += part[4 * cb + j][0][l];
        qs += part[4 * cb + j][1][l];
      }
      v4f rhs;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int t = 4 * kq + i;
        rhs[i] = sbb[rb][t] * (sVb[rb][t][16 * cb + r] - sgam[db][t] * ks[i]);
      }
      const v4f rop = tile_to_operand(rhs);
      v4f dl = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int m = 0; m < 4; m++) dl = mfma4(sTb[rb][r][4 * m + kq], rop[m], dl);
#pragma unroll
      for (int i = 0; i < 4; i++) sDl[cb][4 * kq + i][r] = dl[i];
      const v4f dop = tile_to_operand(dl);
#pragma unroll
      for (int i = 0; i < 4; i++) oz[i] = sgam[db][4 * kq + i] * qs[i];
#pragma unroll
      for (int m = 0; m < 4; m++) oz = mfma4(sMb[rb][r][4 * m + kq], dop[m], oz);
    } else if (w == 2 && ch + 1 < nch) {
      decays(ch + 1);
    }
    __syncthreads();
    // ---- Z: state update S <- gamma_15 S + sum_t dec_t k_t Delta_t^T; chunk ch + kNB - 1's rows to the free buffer
    {
      const float g15 = sgam[db][kC - 1];
#pragma unroll
      for (int b = 0; b < 2; b++) {
        S[b] *= g15;
#pragma unroll
        for (int m = 0; m < 4; m++) {
          const int t = 4 * m + kq;
          S[b] = mfma4(sdec[db][t] * sKb[rb][t][32 * kb + 16 * b + r], sDl[cb][t][r], S[b]);
        }
      }
    }
    stash((ch + kNB - 1) % kNB);
    // the output stores come after the stash: vector memory counts stores and loads together, so a store issued
    // before it would make the stash wait for the store's completion
    if (dl_wave) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int t = 4 * kq + i;
        if (t < n) o[((size_t)(c0 + t) * H + h) * 128 + col] = oz[i] * scale;
      }
    }
    __syncthreads();
  }
  float* dst = planes + (size_t)pout * plane_sz + ((size_t)h * 128 + col) * 128 + 32 * kb + 4 * kq;
#pragma unroll
  for (int b = 0; b < 2; b++) st4(dst + 16 * b, S[b][0], S[b][1], S[b][2], S[b][3]);
}

}  // namespace
}  // namespace q27h

using namespace q27h;

extern "C" int q27h_gdn_step_chunked(const float* q, const float* k, const float* v, int stride, const float* g,
                                     const float* beta, float* planes, const int* in_plane, float* o, int H, int HK,
                                     int T, float scale, q27h_stream_t s) {
  if (H <= 0 || HK <= 0 || T < 0 || stride < 128 || stride % 4) return fail(Q27H_ERR_SHAPE, "gdn_step_chunked: bad shape");
  if (T == 0) return Q27H_OK;
  if (!q || !k || !v || !g || !beta || !planes || !in_plane || !o) return fail(Q27H_ERR_ARG, "gdn_step_chunked: null pointer");
  if (!aligned16(q) || !aligned16(k) || !aligned16(planes))
    return fail(Q27H_ERR_ARG, "gdn_step_chunked: q, k and planes need 16-byte alignment");
  if (T > 65535 * kC) return fail(Q27H_ERR_SHAPE, "gdn_step_chunked: T too large");
  const hipStream_t st = stream_of(s);
  hipLaunchKernelGGL(gdn_chunk_prep_kernel, dim3(min(H, HK), (T + kC - 1) / kC), dim3(64), 0, st, q, k, stride, g, beta,
                     planes, in_plane, o, H, HK, T);
  if (int e = check_launch("gdn_step_chunked")) return e;
  hipLaunchKernelGGL(gdn_chunk_kernel, dim3(H, 128 / kNC), dim3(512), 0, st, q, k, v, stride, g, beta, planes, in_plane,
                     o, H, HK, T, scale);
  return check_launch("gdn_step_chunked");
}
