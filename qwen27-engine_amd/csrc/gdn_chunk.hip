// Gated-DeltaNet recurrence, prefill (flip) mode, in the chunked form on fp32 matrix cores (gdn_step with flip,
// src/ops.h:40-45, src/ops.cu:449-572). Same inputs, outputs and plane semantics as the sequential kernel
// (gdn_rec.hip); the additions happen in another order, so the results agree with it to fp32 rounding, not bit for bit.
//
// Per value head h and chunk of C = 32 tokens (G_c = g_0 + ... + g_c, gamma_c = e^G_c, D_cs = e^(G_c - G_s)):
//   A     = strictly lower part of beta_c D_cs (k_c . k_s)            (C x C)
//   Tinv  = (I + A)^-1                                                 (unit lower triangular)
//   M     = lower part, diagonal included, of D_cs (q_c . k_s)
//   Delta = Tinv (beta (V - gamma (K S)))                              (C x cols: the tokens' delta vectors)
//   O     = scale (gamma (Q S) + M Delta)
//   S    <- gamma_31 S + sum_s D_31,s k_s Delta_s^T
// which unrolls the per-token rule  delta = (v - e^g S^T k) beta,  S <- e^g S + k delta^T,  o = scale S^T q  over the
// chunk (the sequential kernel's comment gives the per-token form). Tinv is formed by 16 x 16 blocks: the diagonal
// blocks as (I + A_dd)^-1 = (I - A_dd)(I + A_dd^2)(I + A_dd^4)(I + A_dd^8) (A_dd^16 = 0), the lower one as
// -Tinv_11 A_10 Tinv_00.
//
// Two launches. gdn_chunk_prep_kernel (four waves per key head and chunk, all chunks in parallel) forms Tinv and M,
// which do not depend on the state. Their free entries (the strictly lower part of Tinv, 496 values, and the lower
// part of M, 528) fill one 32 x 32 matrix P exactly: P[t][j] = M[t][j] for j <= t, Tinv[j][t] for j > t. P is parked
// where the second launch finds it: for a full chunk in the chunk's own rows of o (one copy per 32-column group of the
// head, in that group's columns), which the recurrence overwrites only with that group's own outputs after reading
// it; for a last, partial chunk in the output state plane (keys 0..31 of the group's 32 columns), written only at the
// very end. gdn_chunk_kernel then walks the chunks of one value head and 32 value columns (grid H x 4, 512 threads):
// wave w holds the state rows 32 (w & 3) .. + 31 of the columns 16 (w >> 2) .. + 15 as two 16 x 16 accumulator tiles
// of v_mfma_f32_16x16x4_f32 (lane l: rows 4 (l / 16) + i, column l % 16). K S and Q S are split over the 4 row groups
// of a column half (their operand steps read keys in the state tile's own row order, so the state never leaves its
// accumulators); Delta and O are formed by one wave per column half, with the 16 x 16 right-hand sides turned into
// MFMA operands by lane swaps and the zero upper blocks of Tinv and M skipped; the update is an MFMA into the state
// tiles. A chunk's rows (k, q, v, g, beta, P) are loaded one chunk ahead into the other of two LDS buffers (two,
// three or four buffers measured the same with 16-token chunks; two leave room for 32-token rows).
#include "q27h_device.h"
#include "q27h_internal.h"

namespace q27h {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
constexpr int kC = 32;     // tokens per chunk
constexpr int kNC = 32;    // value columns per workgroup of the recurrence
constexpr int kKP = 132;   // padded LDS row of a chunk's k / q (floats)
constexpr int kPP = 33;    // padded LDS row of the 32 x 32 matrices
constexpr int kDP = 17;    // padded LDS row of Delta (16 columns)
constexpr int kNB = 2;     // row buffers of the recurrence

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

// G_t = g_0 + ... + g_t (token order) on lane t < 32 (lanes >= 32: the sum of all 32), g[32] in LDS, 16-byte aligned
__device__ __forceinline__ float prefix32(const float* g, int l) {
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

// (I - B)^-1 = (I + B)(I + B^2)(I + B^4)(I + B^8) for a strictly lower 16 x 16 block B (rows of kPP floats in LDS),
// by one wave, in registers: every product Z = X Y is formed with its transpose (Z^T = Y^T X^T, a second MFMA chain),
// both turned into B-operand tiles, so the next product reads both operands from registers (the A operand of X is the
// B operand of X^T). Result in the accumulator layout.
__device__ __forceinline__ v4f unit_lower_inverse(const float (*B)[kPP], int r, int kq) {
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

// ---------------------------------------------------------------- prep: P (Tinv and M) of every chunk
// Four waves per (key head, chunk): the 16 x 16 blocks (0, 0), (1, 0), (1, 1) of K K^T and Q K^T once (waves 0, 1,
// 2), then per value head on that key head (their g and beta differ): -A and M by the same waves, the diagonal
// blocks of Tinv on waves 0 and 2, the lower block on wave 1, P assembled in LDS and written out by all 256 threads.
// 34 KB of LDS and at most 128 registers per lane let four workgroups share a CU, so the grid of 2048-token layers
// (16 key heads x 64 chunks) is resident at once: 25.4 us against 31.5 us at three per CU, where the grid ran as two
// successive waves of workgroups. The kernel moves 84 MB (k and q rows in, four copies of P out), about 14 us of HBM
// time.
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4)))
gdn_chunk_prep_kernel(const float* __restrict__ q, const float* __restrict__ k, int stride, const float* __restrict__ g,
                      const float* __restrict__ beta, float* __restrict__ planes, const int* __restrict__ in_plane,
                      float* __restrict__ o, int H, int HK, int T) {
  // the chunk's k and q rows; once the grams are formed the same LDS holds -A (strictly lower), the diagonal blocks
  // of Tinv and P (34 KB in all: four workgroups per CU)
  __shared__ __align__(16) float smem[2 * kC * kKP];
  __shared__ __align__(16) float sg[kC];
  __shared__ float sb[kC];
  float(*sK)[kKP] = (float(*)[kKP])smem;
  float(*sQ)[kKP] = (float(*)[kKP])(smem + kC * kKP);
  float(*sB)[kPP] = (float(*)[kPP])smem;
  float(*sX)[kPP] = (float(*)[kPP])(smem + kC * kPP);
  float(*sP)[kPP] = (float(*)[kPP])(smem + 2 * kC * kPP);
  const int kh = blockIdx.x, c = blockIdx.y;
  const int c0 = c * kC, n = min(kC, T - c0);
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, r = l & 15, kq = l >> 4;
  // g and beta of value head hh (wave 0, one token per lane), loaded a value head ahead of their use
  float pg = 0.0f, pb = 0.0f;
  auto fetch_gb = [&](int hh) {
    if (w == 0 && l < kC) {
      pg = hh < H && l < n ? g[(size_t)(c0 + l) * H + hh] : 0.0f;
      pb = hh < H && l < n ? beta[(size_t)(c0 + l) * H + hh] : 0.0f;
    }
  };
  fetch_gb(kh);
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int e = tid + 256 * j, t = e >> 5, e4 = (e & 31) * 4;
    float4 kv4 = make_float4(0.f, 0.f, 0.f, 0.f), qv4 = kv4;
    if (t < n) {
      kv4 = ld4(k + (size_t)(c0 + t) * stride + kh * 128 + e4);
      qv4 = ld4(q + (size_t)(c0 + t) * stride + kh * 128 + e4);
    }
    *(float4*)&sK[t][e4] = kv4;
    *(float4*)&sQ[t][e4] = qv4;
  }
  __syncthreads();
  // this wave's block (ti, tj) of the 32 x 32 lower part: wave 0 (0, 0), wave 1 (1, 0), wave 2 (1, 1)
  const int ti = w == 0 ? 0 : 1, tj = w == 2 ? 1 : 0;
  v4f kk = {0.f, 0.f, 0.f, 0.f}, qk = kk;
  if (w < 3) {
    kk = gram16(sK + 16 * ti, sK + 16 * tj, r, kq);
    qk = gram16(sQ + 16 * ti, sK + 16 * tj, r, kq);
  }
  const size_t plane_sz = (size_t)H * 128 * 128;
  const int pout = *in_plane == 0 ? 1 : 0;
  for (int h = kh; h < H; h += HK) {
    if (w == 0 && l < kC) {
      sg[l] = pg;
      sb[l] = pb;
    }
    fetch_gb(h + HK);
    __syncthreads();  // also: every wave's gram reads of the k / q rows are done before -A overwrites them
    if (w < 3) {
      const float Gt = prefix32(sg, l);
      const int ss = 16 * tj + r;
      const float Gs = __shfl(Gt, ss, 64);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int cc = 16 * ti + 4 * kq + i;
        const float Gc = __shfl(Gt, cc, 64);  // every lane takes part (a lane exchange reads from active lanes only)
        const float d = ss <= cc ? q27_expf(Gc - Gs) : 0.0f;
        sB[cc][ss] = ss < cc ? -((sb[cc] * d) * kk[i]) : 0.0f;
        sP[cc][ss] = ss <= cc ? d * qk[i] : 0.0f;  // M; the strictly upper entries of the diagonal blocks follow
      }
    }
    __syncthreads();
    if (w == 0 || w == 2) {  // Tinv_dd = (I - B_dd)^-1 (B = -A); its transpose into the strictly upper part of P
      const int d0 = w == 0 ? 0 : 16;
      const v4f x = unit_lower_inverse((const float(*)[kPP]) & sB[d0][d0], r, kq);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int a = 4 * kq + i;
        sX[d0 + a][d0 + r] = x[i];
        if (a > r) sP[d0 + r][d0 + a] = x[i];
      }
    }
    __syncthreads();
    if (w == 1) {  // Tinv_10 = -Tinv_11 A_10 Tinv_00 = Tinv_11 (B_10 Tinv_00); its transpose is P's block (0, 1)
      v4f y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int m = 0; m < 4; m++) y = mfma4(sB[16 + r][4 * m + kq], sX[4 * m + kq][r], y);
      const v4f yop = tile_to_operand(y);
      v4f x = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int m = 0; m < 4; m++) x = mfma4(sX[16 + r][16 + 4 * m + kq], yop[m], x);
#pragma unroll
      for (int i = 0; i < 4; i++) sP[r][16 + 4 * kq + i] = x[i];
    }
    __syncthreads();
    if (n == kC) {  // rows c0 .. c0 + 31 of o, one copy per 32-column group
#pragma unroll
      for (int cg = 0; cg < 128 / kNC; cg++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int t = (tid >> 5) + 8 * j, col = tid & 31;
          o[((size_t)(c0 + t) * H + h) * 128 + kNC * cg + col] = sP[t][col];
        }
    } else {  // keys 0 .. 31 of each column of the output plane (column 32 cg + j holds P[.][j])
#pragma unroll
      for (int cg = 0; cg < 128 / kNC; cg++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int jj = (tid >> 5) + 8 * j, t = tid & 31;
          planes[(size_t)pout * plane_sz + ((size_t)h * 128 + kNC * cg + jj) * 128 + t] = sP[t][jj];
        }
    }
    __syncthreads();  // sg, sb, sB, sX and sP are refilled for the next value head
  }
}

// ---------------------------------------------------------------- the recurrence over the chunks
__global__ void __launch_bounds__(512) gdn_chunk_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                        const float* __restrict__ v, int stride,
                                                        const float* __restrict__ g, const float* __restrict__ beta,
                                                        float* __restrict__ planes, const int* __restrict__ in_plane,
                                                        float* __restrict__ o, int H, int HK, int T, float scale) {
  // a chunk's rows, two buffers (chunk n in use, n + 1 arriving)
  __shared__ __align__(16) float sKb[kNB][kC][kKP];
  __shared__ __align__(16) float sQb[kNB][kC][kKP];
  __shared__ float sVb[kNB][kC][kNC];
  __shared__ __align__(16) float sgb[kNB][kC];
  __shared__ float sbb[kNB][kC];
  __shared__ float sTb[kNB][kC][kPP], sMb[kNB][kC][kPP];  // Tinv and M, unpacked from P
  __shared__ float sgam[2][kC], sdec[2][kC];              // decays of chunks n and n + 1
  __shared__ __align__(16) v4f part[8][4][64];            // K S, Q S partial tiles (two token tiles each)
  __shared__ float sDl[2][kC][kDP];                       // Delta of the two column halves
  const int h = blockIdx.x, kh = h % HK, cg = blockIdx.y;
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, r = l & 15, kq = l >> 4;
  const int kb = w & 3, cb = w >> 2;
  // Delta of column half 0 on wave 0, of half 1 on wave 5 (waves w and w + 4 share a SIMD: SIMDs 0 and 1); the
  // output tiles (token tile (w & 3) - 2 of half w >> 2) on waves 2, 3, 6, 7 (SIMDs 2 and 3); decays on wave 1
  const bool dl_wave = w == 0 || w == 5, o_wave = (w & 3) >= 2;
  const int ot = (w & 3) - 2;
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
  // staging: thread tid takes tokens st_t and st_t + 16, k / q elements st_e4 .. + 3, value / P column st_c
  const int st_t = tid >> 5, st_e4 = (tid & 31) * 4, st_c = tid & 31;
  float4 pk[2], pq[2];
  float pv[2], pt[2], pg = 0.0f, pb = 0.0f;
  auto fetch = [&](int ch) {  // chunk ch's rows into registers (zeros, and no loads, past T)
    const int c0 = ch * kC, n = min(kC, T - c0);
#pragma unroll
    for (int u = 0; u < 2; u++) {
      const int t = st_t + 16 * u;
      pk[u] = make_float4(0.f, 0.f, 0.f, 0.f);
      pq[u] = pk[u];
      pv[u] = 0.0f;
      pt[u] = 0.0f;
      if (t < n) {
        pk[u] = ld4(k + (size_t)(c0 + t) * stride + kh * 128 + st_e4);
        pq[u] = ld4(q + (size_t)(c0 + t) * stride + kh * 128 + st_e4);
        pv[u] = v[(size_t)(c0 + t) * stride + h * 128 + cg * kNC + st_c];
      }
      if (n == kC) pt[u] = o[((size_t)(c0 + t) * H + h) * 128 + cg * kNC + st_c];  // P, parked in o
      else if (n > 0) pt[u] = planes[(size_t)pout * plane_sz + ((size_t)h * 128 + cg * kNC + st_c) * 128 + t];
    }
    if (w == 1 && l < kC) {
      pg = l < n ? g[(size_t)(c0 + l) * H + h] : 0.0f;
      pb = l < n ? beta[(size_t)(c0 + l) * H + h] : 0.0f;
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int u = 0; u < 2; u++) {
      const int t = st_t + 16 * u, j = st_c;
      *(float4*)&sKb[buf][t][st_e4] = pk[u];
      *(float4*)&sQb[buf][t][st_e4] = pq[u];
      sVb[buf][t][j] = pv[u];
      sMb[buf][t][j] = j <= t ? pt[u] : 0.0f;                        // M[t][j]
      sTb[buf][j][t] = j > t ? pt[u] : (j == t ? 1.0f : 0.0f);       // Tinv[j][t]
    }
    if (w == 1 && l < kC) {
      sgb[buf][l] = pg;
      sbb[buf][l] = pb;
    }
  };
  // gamma_t = e^G_t and dec_t = e^(G_31 - G_t) of a chunk, by wave 1 from the g it stashed itself
  auto decays = [&](int buf, int db) {
    const float Gt = prefix32(sgb[buf], l);
    const float G31 = __shfl(Gt, kC - 1, 64);
    if (l < kC) {
      sgam[db][l] = q27_expf(Gt);
      sdec[db][l] = q27_expf(G31 - Gt);
    }
  };

  fetch(0);
  stash(0);
  if (w == 1) decays(0, 0);
  __syncthreads();

  for (int ch = 0; ch < nch; ch++) {
    const int c0 = ch * kC, n = min(kC, T - c0);
    const int rb = ch % kNB, db = ch & 1;
    // chunk ch + 1, in flight during this chunk and stored at its end (past the last chunk: no loads, zeros into the
    // buffer no later chunk reads; unconditional, which keeps the compiler's memory-counter waits exact)
    fetch(ch + 1);
    // partial products X S (X = K rows or Q rows of chunk ch) over this wave's 32 state rows, into part[w][slot ..]
    auto partial = [&](const float (*X)[kKP], int slot) {
      v4f acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
      for (int b = 0; b < 2; b++)
#pragma unroll
        for (int tt = 0; tt < 2; tt++) {
          const float4 x4 = *(const float4*)&X[16 * tt + r][32 * kb + 16 * b + 4 * kq];
          const float xr[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
          for (int i = 0; i < 4; i++) acc[tt] = mfma4(xr[i], S[b][i], acc[tt]);
        }
#pragma unroll
      for (int tt = 0; tt < 2; tt++) part[w][slot + tt][l] = acc[tt];
    };
    // ---- X: partial K S, Q S of chunk ch over this wave's 32 state rows
    partial(sKb[rb], 0);
    partial(sQb[rb], 2);
    __syncthreads();
    // ---- Y: Delta = Tinv (beta (V - gamma K S)) (one wave per column half)
    if (dl_wave) {
      v4f ks[2];
#pragma unroll
      for (int tt = 0; tt < 2; tt++) {
        ks[tt] = part[4 * cb][tt][l];
#pragma unroll
        for (int j = 1; j < 4; j++) ks[tt] += part[4 * cb + j][tt][l];
      }
      v4f rop[2];
#pragma unroll
      for (int tt = 0; tt < 2; tt++) {
        v4f rhs;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int t = 16 * tt + 4 * kq + i;
          rhs[i] = sbb[rb][t] * (sVb[rb][t][16 * cb + r] - sgam[db][t] * ks[tt][i]);
        }
        rop[tt] = tile_to_operand(rhs);
      }
      // Delta_0 = Tinv_00 rhs_0, Delta_1 = Tinv_10 rhs_0 + Tinv_11 rhs_1
      v4f d0 = {0.f, 0.f, 0.f, 0.f}, d1 = d0;
#pragma unroll
      for (int m = 0; m < 4; m++) {
        d0 = mfma4(sTb[rb][r][4 * m + kq], rop[0][m], d0);
        d1 = mfma4(sTb[rb][16 + r][4 * m + kq], rop[0][m], d1);
      }
#pragma unroll
      for (int m = 0; m < 4; m++) d1 = mfma4(sTb[rb][16 + r][16 + 4 * m + kq], rop[1][m], d1);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        sDl[cb][4 * kq + i][r] = d0[i];
        sDl[cb][16 + 4 * kq + i][r] = d1[i];
      }
    }
    __syncthreads();
    // ---- Z: state update S <- gamma_31 S + sum_t dec_t k_t Delta_t^T; output tile O_ot = gamma Q S + M Delta
    //      (O_0 = gamma Q S_0 + M_00 Delta_0, O_1 = gamma Q S_1 + M_10 Delta_0 + M_11 Delta_1; Delta read from LDS
    //      in the B-operand layout); chunk ch + 1's rows to the free buffer, its decays
    v4f oz;  // the output tile (o waves), stored after the stash
    if (o_wave) {
      v4f qs = part[4 * cb][2 + ot][l];
#pragma unroll
      for (int j = 1; j < 4; j++) qs += part[4 * cb + j][2 + ot][l];
#pragma unroll
      for (int i = 0; i < 4; i++) oz[i] = sgam[db][16 * ot + 4 * kq + i] * qs[i];
#pragma unroll
      for (int m = 0; m < 4; m++) oz = mfma4(sMb[rb][16 * ot + r][4 * m + kq], sDl[cb][4 * m + kq][r], oz);
      if (ot == 1) {
#pragma unroll
        for (int m = 0; m < 4; m++) oz = mfma4(sMb[rb][16 + r][16 + 4 * m + kq], sDl[cb][16 + 4 * m + kq][r], oz);
      }
    }
    {
      const float g31 = sgam[db][kC - 1];
#pragma unroll
      for (int b = 0; b < 2; b++) {
        S[b] *= g31;
#pragma unroll
        for (int m = 0; m < kC / 4; m++) {
          const int t = 4 * m + kq;
          S[b] = mfma4(sdec[db][t] * sKb[rb][t][32 * kb + 16 * b + r], sDl[cb][t][r], S[b]);
        }
      }
    }
    stash((ch + 1) % kNB);
    if (w == 1) decays((ch + 1) % kNB, db ^ 1);
    // the output stores come after the stash: vector memory counts stores and loads together, so a store issued
    // before it would make the stash wait for the store's completion
    if (o_wave) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int t = 16 * ot + 4 * kq + i;
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

// The chunked form parks each chunk's matrices in o's rows before the outputs overwrite them, so o may share no
// byte with what the launches read: the q / k / v rows, g, beta and the four state planes.
bool q27h::gdn_chunk_o_overlaps(const float* q, const float* k, const float* v, int stride, const float* g,
                                const float* beta, const float* planes, const float* o, int H, int HK, int T) {
  const size_t fb = sizeof(float);
  const size_t rows = (size_t)(T - 1) * stride;
  const size_t ob = (size_t)T * H * 128 * fb;
  return overlaps(o, ob, q, (rows + (size_t)HK * 128) * fb) || overlaps(o, ob, k, (rows + (size_t)HK * 128) * fb) ||
         overlaps(o, ob, v, (rows + (size_t)H * 128) * fb) || overlaps(o, ob, g, (size_t)T * H * fb) ||
         overlaps(o, ob, beta, (size_t)T * H * fb) || overlaps(o, ob, planes, (size_t)4 * H * 128 * 128 * fb);
}

extern "C" int q27h_gdn_step_chunked(const float* q, const float* k, const float* v, int stride, const float* g,
                                     const float* beta, float* planes, const int* in_plane, float* o, int H, int HK,
                                     int T, float scale, q27h_stream_t s) {
  if (H <= 0 || HK <= 0 || T < 0 || stride < 128 || stride % 4) return fail(Q27H_ERR_SHAPE, "gdn_step_chunked: bad shape");
  if (T == 0) return Q27H_OK;
  if (!q || !k || !v || !g || !beta || !planes || !in_plane || !o) return fail(Q27H_ERR_ARG, "gdn_step_chunked: null pointer");
  if (!aligned16(q) || !aligned16(k) || !aligned16(planes))
    return fail(Q27H_ERR_ARG, "gdn_step_chunked: q, k and planes need 16-byte alignment");
  if (T > 65535 * kC) return fail(Q27H_ERR_SHAPE, "gdn_step_chunked: T too large");
  if (gdn_chunk_o_overlaps(q, k, v, stride, g, beta, planes, o, H, HK, T))
    return fail(Q27H_ERR_ARG, "gdn_step_chunked: o overlaps q / k / v rows, g, beta or the state planes");
  const hipStream_t st = stream_of(s);
  hipLaunchKernelGGL(gdn_chunk_prep_kernel, dim3(min(H, HK), (T + kC - 1) / kC), dim3(256), 0, st, q, k, stride, g, beta,
                     planes, in_plane, o, H, HK, T);
  if (int e = check_launch("gdn_step_chunked")) return e;
  hipLaunchKernelGGL(gdn_chunk_kernel, dim3(H, 128 / kNC), dim3(512), 0, st, q, k, v, stride, g, beta, planes, in_plane,
                     o, H, HK, T, scale);
  return check_launch("gdn_step_chunked");
}
