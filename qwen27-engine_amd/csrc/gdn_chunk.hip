// Gated-DeltaNet recurrence, prefill (flip) mode, in the chunked form on fp32 matrix cores (gdn_step with flip,
// src/ops.h:40-45, src/ops.cu:449-572). Same inputs, outputs and plane semantics as the sequential kernel
// (gdn_rec.hip); the additions happen in another order, so the results agree with it to fp32 rounding, not bit for bit.
//
// Per value head h and chunk of C = 16 tokens (G_c = g_0 + ... + g_c, gamma_c = e^G_c, D_cs = e^(G_c - G_s)):
//   A     = strictly lower part of beta_c D_cs (k_c . k_s)            (C x C)
//   Tinv  = (I + A)^-1 = (I - A)(I + A^2)(I + A^4)(I + A^8)          (A^16 = 0)
//   Delta = Tinv (beta (V - gamma (K S)))                              (C x cols: the tokens' delta vectors)
//   O     = scale (gamma (Q S) + (lower part incl. diagonal of D (Q K^T)) Delta)
//   S    <- gamma_15 S + sum_s D_15,s k_s Delta_s^T
// which unrolls the per-token rule  delta = (v - e^g S^T k) beta,  S <- e^g S + k delta^T,  o = scale S^T q  over the
// chunk (the sequential kernel's comment gives the per-token form).
//
// gfx950 layout: a 512-thread workgroup = one value head and 32 value columns (grid H x 4); wave w holds the state
// rows 32 (w & 3) .. + 31 of the columns 16 (w >> 2) .. + 15 of the workgroup as two 16 x 16 accumulator tiles of
// v_mfma_f32_16x16x4_f32 (lane l: rows 4 (l / 16) + i, column l % 16). Every product is a 16 x 16 x 4 MFMA: K K^T and
// Q K^T split over the 8 waves by key (16 keys each), K S and Q S over the 4 row groups of a column half, the 16 x 16
// products of the inverse on one wave. Operands whose rows are the MFMA's K dimension are read in the state tile's
// own row order (key 16 b + 4 (l / 16) + i at step i), so the state is never moved out of its accumulators.
#include "q27h_device.h"
#include "q27h_internal.h"

namespace q27h {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
constexpr int kC = 16;     // tokens per chunk
constexpr int kNC = 32;    // value columns per workgroup
constexpr int kKP = 132;   // padded LDS row of the chunk's k / q (floats)
constexpr int kMP = 17;    // padded LDS row of the 16 x 16 matrices

__device__ __forceinline__ v4f mfma4(float a, float b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// LDS writes of this wave visible to its own later LDS reads (other lanes' addresses)
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Z = (X + ix I)(Y + iy I) for 16 x 16 matrices in LDS, by one wave; Z in the accumulator layout.
__device__ __forceinline__ v4f mm16(const float (*X)[kMP], const float (*Y)[kMP], bool ix, bool iy, int l) {
  const int r = l & 15, kq = l >> 4;
  v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int m = 0; m < 4; m++) {
    const int kk = 4 * m + kq;
    const float a = X[r][kk] + (ix && r == kk ? 1.0f : 0.0f);
    const float b = Y[kk][r] + (iy && r == kk ? 1.0f : 0.0f);
    acc = mfma4(a, b, acc);
  }
  return acc;
}
__device__ __forceinline__ void put16(float (*Z)[kMP], v4f z, int l) {
  const int r = l & 15, kq = l >> 4;
#pragma unroll
  for (int i = 0; i < 4; i++) Z[4 * kq + i][r] = z[i];
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

__global__ void __launch_bounds__(512) gdn_chunk_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                        const float* __restrict__ v, int stride,
                                                        const float* __restrict__ g, const float* __restrict__ beta,
                                                        float* __restrict__ planes, const int* __restrict__ in_plane,
                                                        float* __restrict__ o, int H, int HK, int T, float scale) {
  // chunk rows, four buffers (chunk n in use, n + 1 and n + 2 being prepared, n + 3 arriving)
  __shared__ __align__(16) float sKb[4][kC][kKP];
  __shared__ __align__(16) float sQb[4][kC][kKP];
  __shared__ float sVb[4][kC][kNC];
  __shared__ float sgb[4][kC], sbb[4][kC];
  // state-independent results of a chunk: decays and M (made two chunks ahead, three buffers), B (two ahead, read
  // one ahead), Tinv (one ahead)
  __shared__ float sgam[3][kC], sdec[3][kC], sG[kC];
  __shared__ float sB[2][kC][kMP], sM[3][kC][kMP], sT[2][kC][kMP];
  __shared__ __align__(16) v4f part[8][2][64];   // K S, Q S partial tiles of chunk n
  __shared__ __align__(16) v4f part2[8][2][64];  // K K^T, Q K^T partial tiles of chunk n + 2
  __shared__ float sB2[kC][kMP], sB4[kC][kMP], sB8[kC][kMP], sP[kC][kMP];  // the inverse's products
  __shared__ float sDl[2][kC][kMP];
  const int h = blockIdx.x, kh = h % HK, cg = blockIdx.y;
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, r = l & 15, kq = l >> 4;
  const int kb = w & 3, cb = w >> 2;
  const int col = cg * kNC + cb * 16 + r;  // this lane's value column (state tile column)
  const size_t plane_sz = (size_t)H * 128 * 128;
  const int pin = *in_plane;
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
  float pv, pg = 0.0f, pb = 0.0f;
  auto fetch = [&](int ch) {  // chunk ch's rows into registers (zeros, and no loads, past T)
    const int c0 = ch * kC, n = min(kC, T - c0);
    pk = make_float4(0.f, 0.f, 0.f, 0.f);
    pq = pk;
    pv = 0.0f;
    if (st_t < n) {
      pk = ld4(k + (size_t)(c0 + st_t) * stride + kh * 128 + st_e4);
      pq = ld4(q + (size_t)(c0 + st_t) * stride + kh * 128 + st_e4);
      pv = v[(size_t)(c0 + st_t) * stride + h * 128 + cg * kNC + st_c];
    }
    if (tid < kC) {
      pg = tid < n ? g[(size_t)(c0 + tid) * H + h] : 0.0f;
      pb = tid < n ? beta[(size_t)(c0 + tid) * H + h] : 0.0f;
    }
  };
  auto stash = [&](int buf) {
    *(float4*)&sKb[buf][st_t][st_e4] = pk;
    *(float4*)&sQb[buf][st_t][st_e4] = pq;
    sVb[buf][st_t][st_c] = pv;
    if (tid < kC) {
      sgb[buf][tid] = pg;
      sbb[buf][tid] = pb;
    }
  };
  // decays of chunk ch (wave 7): G = prefix sum of g in token order, gamma = e^G, dec = e^(G_15 - G)
  auto decays = [&](int ch) {
    if (w == 7) {
      const int rb = ch & 3, db = ch % 3;
      float Gt = 0.0f;
#pragma unroll
      for (int j = 0; j < kC; j++) Gt += j <= l ? sgb[rb][j] : 0.0f;
      const float G15 = __shfl(Gt, kC - 1, 64);
      if (l < kC) {
        sG[l] = Gt;
        sgam[db][l] = q27_expf(Gt);
        sdec[db][l] = q27_expf(G15 - Gt);
      }
    }
  };
  // partial K K^T and Q K^T of chunk ch over this wave's 16 keys
  auto kk_part = [&](int ch) {
    const int rb = ch & 3;
    v4f kk = {0.f, 0.f, 0.f, 0.f}, qk = kk;
#pragma unroll
    for (int m = 0; m < 4; m++) {
      const int key = 16 * w + 4 * m + kq;
      const float kr = sKb[rb][r][key];
      kk = mfma4(kr, kr, kk);
      qk = mfma4(sQb[rb][r][key], kr, qk);
    }
    part2[w][0][l] = kk;
    part2[w][1][l] = qk;
  };
  // B = -A from K K^T and M from Q K^T of chunk ch (elements e0, e0 + step, ... of the 512)
  auto reduce_bm = [&](int ch, int e0, int step) {
    const int rb = ch & 3, pb2 = ch & 1, db = ch % 3;
    for (int e = e0; e < 512; e += step) {
      const int which = e >> 8, c = (e >> 4) & 15, s = e & 15;
      const int L = 16 * (c >> 2) + s, i = c & 3;  // accumulator position of element (c, s)
      float acc = 0.0f;
#pragma unroll
      for (int ww = 0; ww < 8; ww++) acc += part2[ww][which][L][i];
      const float d = s <= c ? q27_expf(sG[c] - sG[s]) : 0.0f;
      if (which == 0) sB[pb2][c][s] = s < c ? -((sbb[rb][c] * d) * acc) : 0.0f;
      else sM[db][c][s] = s <= c ? d * acc : 0.0f;
    }
  };
  // Tinv of chunk ch = (I + B)(I + B^2)(I + B^4)(I + B^8), by one wave
  auto inverse = [&](int ch) {
    const int pb2 = ch & 1;
    put16(sB2, mm16(sB[pb2], sB[pb2], false, false, l), l);
    wave_lds_sync();
    put16(sB4, mm16(sB2, sB2, false, false, l), l);
    put16(sP, mm16(sB[pb2], sB2, true, true, l), l);
    wave_lds_sync();
    put16(sB8, mm16(sB4, sB4, false, false, l), l);
    put16(sB2, mm16(sP, sB4, false, true, l), l);  // (I + B)(I + B^2)(I + B^4)
    wave_lds_sync();
    put16(sT[pb2], mm16(sB2, sB8, false, true, l), l);
  };

  // prologue: rows of chunks 0..2; decays, B, M of chunks 0 and 1; Tinv of chunk 0
  for (int c = 0; c < 3; c++) {
    fetch(c);
    stash(c);
  }
  __syncthreads();
  for (int c = 0; c < 2 && c < nch; c++) {
    decays(c);
    kk_part(c);
    __syncthreads();
    reduce_bm(c, tid, 512);
    __syncthreads();
  }
  if (w == 1) inverse(0);
  __syncthreads();

  for (int ch = 0; ch < nch; ch++) {
    const int c0 = ch * kC, n = min(kC, T - c0);
    const int rb = ch & 3, db = ch % 3, pb2 = ch & 1;
    // rows of chunk ch + 3, in flight during this chunk and stored at its end (past the last chunk: no loads, zeros
    // into a buffer no later chunk reads; unconditional, which keeps the compiler's memory-counter waits exact)
    fetch(ch + 3);
    // ---- X: partial K S, Q S of chunk ch; partial K K^T, Q K^T and the decays of chunk ch + 2
    {
      v4f ks = {0.f, 0.f, 0.f, 0.f}, qs = ks;
#pragma unroll
      for (int b = 0; b < 2; b++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int key = 32 * kb + 16 * b + 4 * kq + i;
          ks = mfma4(sKb[rb][r][key], S[b][i], ks);
          qs = mfma4(sQb[rb][r][key], S[b][i], qs);
        }
      }
      part[w][0][l] = ks;
      part[w][1][l] = qs;
    }
    if (ch + 2 < nch) {
      kk_part(ch + 2);
      decays(ch + 2);
    }
    __syncthreads();
    // ---- Y: waves 0 and 4 (one per column half): Delta = Tinv (beta (V - gamma K S)), O = gamma Q S + M Delta;
    //      wave 1: Tinv of chunk ch + 1; waves 2, 3, 5, 6, 7: B and M of chunk ch + 2
    v4f oz;  // this chunk's output tile (waves 0 and 4), stored at the end of the chunk
    if (kb == 0) {
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
      for (int m = 0; m < 4; m++) dl = mfma4(sT[pb2][r][4 * m + kq], rop[m], dl);
      put16(sDl[cb], dl, l);
      const v4f dop = tile_to_operand(dl);
#pragma unroll
      for (int i = 0; i < 4; i++) oz[i] = sgam[db][4 * kq + i] * qs[i];
#pragma unroll
      for (int m = 0; m < 4; m++) oz = mfma4(sM[db][r][4 * m + kq], dop[m], oz);
    } else if (w == 1) {
      if (ch + 1 < nch) inverse(ch + 1);
    } else if (ch + 2 < nch) {
      const int slot = (w < 4 ? w - 2 : w - 3) * 64 + l;  // 0..319 over waves 2, 3, 5, 6, 7
      reduce_bm(ch + 2, slot, 320);
    }
    __syncthreads();
    // ---- Z: state update S <- gamma_15 S + sum_t dec_t k_t Delta_t^T; chunk ch + 3's rows to the free buffer
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
    stash((ch + 3) & 3);
    // the output stores come after the stash: vector memory counts stores and loads together, so a store issued
    // before it would make the stash wait for the store's completion
    if (kb == 0) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int t = 4 * kq + i;
        if (t < n) o[((size_t)(c0 + t) * H + h) * 128 + col] = oz[i] * scale;
      }
    }
    __syncthreads();
  }
  float* dst = planes + (size_t)(pin == 0 ? 1 : 0) * plane_sz + ((size_t)h * 128 + col) * 128 + 32 * kb + 4 * kq;
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
  hipLaunchKernelGGL(gdn_chunk_kernel, dim3(H, 128 / kNC), dim3(512), 0, stream_of(s), q, k, v, stride, g, beta, planes,
                     in_plane, o, H, HK, T, scale);
  return check_launch("gdn_step_chunked");
}
