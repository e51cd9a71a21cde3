/* CPU oracle for the fused per-layer ops: TEST INFRASTRUCTURE ONLY (see q27_oracle.h).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this file's library, and only
 * as the checker / the CPU baseline. Build: `make -C oracle` (gcc -O2 -ffp-contract=off, no fast math).
 *
 * Reference file:line citations are to avallavall/qwen27-engine. How each function is pinned (the
 * reference ships no golden vectors for this path, so pins are closed forms, special cases, brute force
 * and the reference's own fused == unfused identities; all live in tests/test_oracle_*.py):
 *   q27o_expf, q27o_logf, q27o_sincos  ulp distance to glibc expf/logf and to sin/cos in long double
 *   q27o_f2h / q27o_h2f / q27o_f2bf   exhaustive round trip over all 65536 codes + RNE ties vs numpy
 *   q8_1 (quantize_q8_1, q8_store)    closed-form blocks (zero, one-hot, ties), |q| <= 127, xd = fp16(d)
 *                                     vs numpy float16, roundf(y / d) vs numpy's quotient on near-tie blocks;
 *                                     xs by blocks whose xor 8-4-2-1 sums are derived by hand
 *                                     (tests/treepins.py, test_oracle_trees.py)
 *   rmsnorm / rmsnorm_q8 / sum_norm*  constant-row closed form, mean(h^2) = m/(m+eps) invariant, fused ==
 *                                     unfused chain (tools/test_fused.cu:55-74); the reduction tree (strided
 *                                     per-thread partials, warp and cross-warp butterflies) by rows whose sums of
 *                                     squares are derived by hand for that tree and differ for a sequential sum,
 *                                     a contiguous layout or a reversed per-thread order; (scale * v) * w by
 *                                     integer rows (test_oracle_trees.py)
 *   swiglu(_q8)                       silu(0) = 0, asymptotes, fused == swiglu + quantize_q8_1
 *   gated_rmsnorm(_q8)                w = 1 / large z reduces to RMSNorm, fused == unfused + quantize; the
 *                                     4-warp tree and the product order as for the rows
 *   l2norm_heads, gdn_conv*, gates    sum y^2 = S/(S+eps) per head, fused == unfused, the strided-lane tree
 *                                     (tools/test_fused.cu:76-102), decode == prefill conv on the same rows
 *   attn_prep                         8-warp head-norm tree and (scale * v) * w as for the rows; pair norms
 *                                     preserved by RoPE, p = 0 identity, rope3 with t=h=w == plain
 *                                     positions, q8_0/f16 cache special cases, numpy float64 rotation bound
 *   get_rows_*                        hand-built one-hot blocks decoded by brute force, Q8_0 closed form
 */
#include "q27_oracle.h"

#include <math.h>
#include <stdint.h>
#include <string.h>

/* ------------------------------------------------------------------------------------------------ math
 * expf: Cody-Waite reduction x = k ln2 + r (k = rint(x log2 e), ln2 split in two floats, fmaf), then the
 * degree-7 Taylor polynomial of e^r in Horner form with fmaf, scaled by 2^k with ldexpf (one rounding).
 * |r| <= ln2/2, truncation error < 6e-9 relative. Method: J.-M. Muller, Elementary Functions, ch. 11.
 * The reference uses expf under -use_fast_math (src/ops.cu:52-54); this routine replaces it on both the
 * CPU and the GPU side so the two agree bit for bit. */
float q27o_expf(float x) {
  if (x != x) return x + x;
  if (x > 88.7228394f) return INFINITY;
  if (x < -103.972084f) return 0.0f;
  const float k = rintf(x * 1.44269502f);
  float r = fmaf(-k, 0.693145752f, x);
  r = fmaf(-k, 1.42860677e-06f, r);
  float p = 1.98412698e-4f;
  p = fmaf(p, r, 1.38888889e-3f);
  p = fmaf(p, r, 8.33333333e-3f);
  p = fmaf(p, r, 4.16666667e-2f);
  p = fmaf(p, r, 1.66666667e-1f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return ldexpf(p, (int)k);
}

/* logf: x = 2^e m with m in [sqrt(1/2), sqrt(2)), f = m - 1 (exact), s = f / (2 + f),
 * log m = 2 atanh(s) = 2s + s (2z/3 + 2z^2/5 + 2z^3/7 + 2z^4/9 + 2z^5/11), z = s^2 (|s| < 0.172),
 * log x = e ln2_hi + (e ln2_lo + log m). Method: Muller, Elementary Functions; the same split as fdlibm. */
float q27o_logf(float x) {
  if (x != x || x < 0.0f) return NAN;
  if (x == 0.0f) return -INFINITY;
  if (x == INFINITY) return x;
  int e = 0;
  if (x < 1.17549435e-38f) { x *= 8388608.0f; e = -23; }
  uint32_t ix;
  memcpy(&ix, &x, 4);
  e += (int)((ix >> 23) & 0xff) - 127;
  ix = (ix & 0x007fffffu) | 0x3f800000u;
  float m;
  memcpy(&m, &ix, 4);
  if (m > 1.41421354f) { m *= 0.5f; e += 1; }
  const float f = m - 1.0f;
  const float s = f / (2.0f + f);
  const float z = s * s;
  float R = 1.81818187e-1f;
  R = fmaf(R, z, 2.22222224e-1f);
  R = fmaf(R, z, 2.85714298e-1f);
  R = fmaf(R, z, 4.00000006e-1f);
  R = fmaf(R, z, 6.66666687e-1f);
  R = R * z;
  const float logm = fmaf(s, R, s + s);
  const float fe = (float)e;
  return fmaf(fe, 0.693145752f, fmaf(fe, 1.42860677e-06f, logm));
}

/* sin/cos of a float angle: Cody-Waite reduction in double, theta = k pi/2 + r with pi/2 split in two
 * doubles (33 + 53 bits; k < 2^20 keeps k * pio2_1 exact), Taylor polynomials of sin and cos on
 * |r| <= pi/4 to degree 21 / 20 in double (truncation < 1e-24), then one rounding to float. Plain
 * double multiplies and adds, no fma, so the CPU and the GPU evaluate the same operations.
 * Method: Muller, Elementary Functions, ch. 11 (Cody-Waite); fdlibm __ieee754_rem_pio2 constants. */
void q27o_sincos(float theta, float* s_out, float* c_out) {
  const double th = (double)theta;
  const double kd = rint(th * 6.36619772367581382433e-01);
  const double pio2_1 = 1.57079632673412561417e+00, pio2_1t = 6.07710050650619224932e-11;
  const double r = (th - kd * pio2_1) - kd * pio2_1t;
  const double z = r * r;
  double sp = 1.9572941063391263e-20;          /* 1/21! */
  sp = sp * z + -8.22063524662433e-18;       /* -1/19! */
  sp = sp * z + 2.8114572543455206e-15;        /* 1/17! */
  sp = sp * z + -7.647163731819816e-13;       /* -1/15! */
  sp = sp * z + 1.6059043836821613e-10;        /* 1/13! */
  sp = sp * z + -2.505210838544172e-08;       /* -1/11! */
  sp = sp * z + 2.7557319223985893e-06;        /* 1/9! */
  sp = sp * z + -0.0001984126984126984;       /* -1/7! */
  sp = sp * z + 0.008333333333333333;        /* 1/5! */
  sp = sp * z + -0.16666666666666666;       /* -1/3! */
  const double sn = r + (r * z) * sp;
  double cp = 4.110317623312165e-19;          /* 1/20! */
  cp = cp * z + -1.5619206968586225e-16;       /* -1/18! */
  cp = cp * z + 4.779477332387385e-14;        /* 1/16! */
  cp = cp * z + -1.1470745597729725e-11;       /* -1/14! */
  cp = cp * z + 2.08767569878681e-09;        /* 1/12! */
  cp = cp * z + -2.755731922398589e-07;       /* -1/10! */
  cp = cp * z + 2.48015873015873e-05;        /* 1/8! */
  cp = cp * z + -0.001388888888888889;       /* -1/6! */
  cp = cp * z + 0.041666666666666664;        /* 1/4! */
  cp = cp * z + -0.5;                          /* -1/2! */
  const double cs = 1.0 + z * cp;
  const long long q = (long long)kd & 3;
  double s, c;
  if (q == 0) { s = sn; c = cs; }
  else if (q == 1) { s = cs; c = -sn; }
  else if (q == 2) { s = -sn; c = -cs; }
  else { s = -cs; c = sn; }
  *s_out = (float)s;
  *c_out = (float)c;
}

/* src/ops.cu:52-54 */
float q27o_silu(float x) { return x / (1.0f + q27o_expf(-x)); }
float q27o_sigmoid(float x) { return 1.0f / (1.0f + q27o_expf(-x)); }
float q27o_softplus(float x) { return x > 20.0f ? x : q27o_logf(1.0f + q27o_expf(x)); }

/* IEEE binary16 conversion, round to nearest even with subnormals (the semantics of src/requant.cpp:14-55
 * and of __float2half), written as integer arithmetic on the float's fields. */
uint16_t q27o_f2h(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const uint32_t ex = (u >> 23) & 0xffu, man = u & 0x7fffffu;
  if (ex == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u | (man >> 13) : 0u));
  const int e = (int)ex - 112; /* exponent in half bias */
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return sign;
    const uint32_t full = man | 0x800000u;
    const int sh = 14 - e;
    uint32_t h = full >> sh;
    const uint32_t rem = full & ((1u << sh) - 1u), halfway = 1u << (sh - 1);
    if (rem > halfway || (rem == halfway && (h & 1u))) h++;
    return (uint16_t)(sign | h);
  }
  uint32_t h = ((uint32_t)e << 10) | (man >> 13);
  const uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return (uint16_t)(sign | h);
}

float q27o_h2f(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t ex = (h >> 10) & 0x1fu, man = h & 0x3ffu;
  uint32_t u;
  if (ex == 0) {
    if (man == 0) u = sign;
    else {
      float f = (float)man * 5.96046448e-08f; /* man * 2^-24, exact */
      memcpy(&u, &f, 4);
      u |= sign;
    }
  } else if (ex == 31) u = sign | 0x7f800000u | (man << 13);
  else u = sign | ((ex + 112u) << 23) | (man << 13);
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* __float2bfloat16: round to nearest even, NaN kept quiet. */
uint16_t q27o_f2bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float q27o_bf2f(uint16_t b) {
  const uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* theta of rotary pair j is p * theta_scale^j (src/ops.cu:621); the power is taken once on the host. */
void q27o_rope_freqs(float theta_scale, float* freq32) {
  for (int j = 0; j < 32; j++) freq32[j] = powf(theta_scale, (float)j);
}

/* ------------------------------------------------------------------------------------------------ reductions
 * warp_sum (src/ops.cu:34-38): v += shfl_xor(v, o) for o = 16, 8, 4, 2, 1 over 32 lanes. Every lane ends with
 * the same value; lane 0's is returned. a[] is clobbered. */
static float butterfly(float* a, int width) {
  for (int o = width / 2; o > 0; o >>= 1) {
    float b[32];
    for (int l = 0; l < width; l++) b[l] = a[l] + a[l ^ o];
    memcpy(a, b, sizeof(float) * (size_t)width);
  }
  return a[0];
}

/* block_sum (src/ops.cu:40-50) for a block of B threads (B a multiple of 32, <= 1024) holding part[B]. */
static float block_sum(const float* part, int B) {
  float ws[32];
  const int nw = B / 32;
  for (int w = 0; w < nw; w++) {
    float a[32];
    memcpy(a, part + 32 * w, sizeof a);
    ws[w] = butterfly(a, 32);
  }
  float a[32];
  for (int l = 0; l < 32; l++) a[l] = l < nw ? ws[l] : 0.0f;
  return butterfly(a, 32);
}

/* Per-thread partial sums of squares: thread t of B adds v[i]^2 for i = t, t + B, ... (starting from 0). */
static void thread_sq(const float* v, int n, int B, float* part) {
  for (int t = 0; t < B; t++) {
    float s = 0.0f;
    for (int i = t; i < n; i += B) s += v[i] * v[i];
    part[t] = s;
  }
}

/* q8_store (src/common.cuh:68-87) over one 32-value block starting at flat index i0 (i0 % 32 == 0):
 * amax = max |y|, d = amax / 127, q = amax == 0 ? 0 : (int8)roundf(y / d), xd = fp16(d) as f32; xs per 16 =
 * xor butterfly 8, 4, 2, 1 of the unquantized values. */
static void q8_block(const float* y, int8_t* xq, float* xd, float* xs, size_t i0) {
  float amax = 0.0f;
  for (int l = 0; l < 32; l++) amax = fmaxf(amax, fabsf(y[l]));
  const float d = amax / 127.0f;
  for (int l = 0; l < 32; l++) xq[i0 + l] = amax == 0.0f ? 0 : (int8_t)roundf(y[l] / d);
  xd[i0 / 32] = q27o_h2f(q27o_f2h(d));
  if (xs) {
    for (int hlf = 0; hlf < 2; hlf++) {
      float a[16];
      memcpy(a, y + 16 * hlf, sizeof a);
      xs[i0 / 16 + hlf] = butterfly(a, 16);
    }
  }
}

/* ------------------------------------------------------------------------------------------------ ops */

/* quantize_q8_1 (src/qgemv.cu:817-845): x[c][K] -> xq[c][K], xd[c][K/32], xs[c][K/16]. K % 32 == 0. */
void q27o_quantize_q8_1(const float* x, int8_t* xq, float* xd, int K, int ncols, float* xs) {
  for (size_t i0 = 0; i0 < (size_t)K * (size_t)ncols; i0 += 32) q8_block(x + i0, xq, xd, xs, i0);
}

/* rmsnorm (src/ops.cu:57-68, launch :746-748): block of B = n >= 1024 ? 1024 : 256 threads per row. */
void q27o_rmsnorm(const float* x, const float* w, float* y, int n, int rows, float eps, int ystride) {
  const int B = n >= 1024 ? 1024 : 256;
  const int ys = ystride ? ystride : n;
  float part[1024];
  for (int r = 0; r < rows; r++) {
    const float* xr = x + (size_t)r * n;
    thread_sq(xr, n, B, part);
    const float t = block_sum(part, B);
    const float scale = 1.0f / sqrtf(t / (float)n + eps);
    for (int i = 0; i < n; i++) y[(size_t)r * ys + i] = scale * xr[i] * w[i];
  }
}

/* add / swiglu (src/ops.cu:70-82) */
void q27o_add(const float* x, const float* a, float* y, int n) {
  for (int i = 0; i < n; i++) y[i] = x[i] + a[i];
}
void q27o_swiglu(const float* g, const float* u, float* y, int n) {
  for (int i = 0; i < n; i++) y[i] = q27o_silu(g[i]) * u[i];
}

/* norm_q8_row (src/ops.cu:92-108): RMSNorm of one 5120-row held by 1024 threads (5 values each) -> h, q8_1, xs. */
static void norm_q8_row(const float* v, const float* w, float eps, int n, size_t row, float* h, int8_t* xq, float* xd,
                        float* xs) {
  float part[1024];
  thread_sq(v, n, 1024, part);
  const float t = block_sum(part, 1024);
  const float scale = 1.0f / sqrtf(t / (float)n + eps);
  float y[32];
  for (int b = 0; b < n / 32; b++) {
    for (int l = 0; l < 32; l++) {
      const int i = 32 * b + l;
      y[l] = scale * v[i] * w[i];
      if (h) h[row * (size_t)n + i] = y[l];
    }
    q8_block(y, xq, xd, xs, row * (size_t)n + 32 * (size_t)b);
  }
}

/* rmsnorm_q8 (src/ops.cu:110-121, 697-701); n must be 5120 in the reference (5 values x 1024 threads). */
void q27o_rmsnorm_q8(const float* x, const float* w, float* h, int8_t* xq, float* xd, int n, int rows, float eps, float* xs) {
  for (int r = 0; r < rows; r++) norm_q8_row(x + (size_t)r * n, w, eps, n, (size_t)r, h, xq, xd, xs);
}

/* sum_norm_q8, no exchange (src/ops.cu:251-259): x += partial in place, then norm_q8_row without xs. */
void q27o_sum_norm_q8(float* x, const float* partial, int n, int rows, const float* w, float eps, float* h, int8_t* xq,
                      float* xd) {
  for (int r = 0; r < rows; r++) {
    float* xr = x + (size_t)r * n;
    const float* pr = partial + (size_t)r * n;
    for (int i = 0; i < n; i++) xr[i] = xr[i] + pr[i];
    norm_q8_row(xr, w, eps, n, (size_t)r, h, xq, xd, NULL);
  }
}

/* sum_norm_rows, no exchange (src/prefill.cu:217-265): the same per row, with xs. */
void q27o_sum_norm_rows(float* x, const float* partial, int n, int M, const float* w, float eps, float* h, int8_t* xq,
                        float* xd, float* xs) {
  for (int r = 0; r < M; r++) {
    float* xr = x + (size_t)r * n;
    const float* pr = partial + (size_t)r * n;
    for (int i = 0; i < n; i++) xr[i] = xr[i] + pr[i];
    norm_q8_row(xr, w, eps, n, (size_t)r, h, xq, xd, xs);
  }
}

/* add_norm_rows (src/prefill.cu:419-453): recv null -> x += partial; else x += bf16(partial) + recv. */
void q27o_add_norm_rows(float* x, const float* partial, const uint16_t* recv_bf16, int n, int M, const float* w, float eps,
                        float* h, int8_t* xq, float* xd, float* xs) {
  for (int r = 0; r < M; r++) {
    float* xr = x + (size_t)r * n;
    const float* pr = partial + (size_t)r * n;
    for (int i = 0; i < n; i++) {
      if (recv_bf16)
        xr[i] = xr[i] + (q27o_bf2f(q27o_f2bf(pr[i])) + q27o_bf2f(recv_bf16[(size_t)r * n + i]));
      else
        xr[i] = xr[i] + pr[i];
    }
    norm_q8_row(xr, w, eps, n, (size_t)r, h, xq, xd, xs);
  }
}

/* gemv_bf16_pair (src/ops.cu:377-393): per output row of [Wa; Wb] and token, 256 threads; thread v adds
 * (w[k] x[k] + w[k + 1] x[k + 1]) for k = 2v, 2v + 512, ... < K, then block_sum. */
void q27o_gemv_bf16_pair(const uint16_t* Wa, const uint16_t* Wb, const float* x, float* ya, float* yb, int N, int K, int T) {
  float part[256];
  for (int t = 0; t < T; t++)
    for (int row = 0; row < 2 * N; row++) {
      const uint16_t* w = row < N ? Wa + (size_t)row * K : Wb + (size_t)(row - N) * K;
      const float* xt = x + (size_t)t * K;
      for (int v = 0; v < 256; v++) {
        float acc = 0.0f;
        for (int k = 2 * v; k < K; k += 512) acc = acc + (q27o_bf2f(w[k]) * xt[k] + q27o_bf2f(w[k + 1]) * xt[k + 1]);
        part[v] = acc;
      }
      const float y = block_sum(part, 256);
      if (row < N) ya[(size_t)t * N + row] = y;
      else yb[(size_t)t * N + row - N] = y;
    }
}

/* ---------------------------------------------------------------- wire formats of the two-card sum
 * to_bf16 (src/prefill.cu:338-345): y = bf16(x), round to nearest even. */
void q27o_to_bf16(const float* x, uint16_t* y, size_t n) {
  for (size_t i = 0; i < n; i++) y[i] = q27o_f2bf(x[i]);
}

/* to_q8_wire (src/prefill.cu:347-370): per row of n values, y = partial (+ ef unless first); per block of qb values
 * amax, d = amax / 127, q = amax == 0 ? 0 : roundf(y / d), scale fp16(d); ef = y - fp16(d) * q (a product, then a
 * difference: no contraction). Row layout: n int8 values, then n / qb fp16 scales. */
void q27o_to_q8_wire(const float* partial, float* ef, int first, uint8_t* wire, int n, int M, int qb) {
  const size_t rb = (size_t)n + 2 * (size_t)n / qb;
  for (int r = 0; r < M; r++) {
    int8_t* q8 = (int8_t*)(wire + r * rb);
    uint8_t* sc = wire + r * rb + n;
    for (int b = 0; b < n / qb; b++) {
      float y[32];
      float amax = 0.0f;
      for (int l = 0; l < qb; l++) {
        const size_t i = (size_t)r * n + (size_t)b * qb + l;
        y[l] = ef && !first ? partial[i] + ef[i] : partial[i];
        amax = fmaxf(amax, fabsf(y[l]));
      }
      const float d = amax / 127.0f;
      const uint16_t dh = q27o_f2h(d);
      sc[2 * b] = (uint8_t)(dh & 0xff);
      sc[2 * b + 1] = (uint8_t)(dh >> 8);
      for (int l = 0; l < qb; l++) {
        const int q = amax == 0.0f ? 0 : (int)roundf(y[l] / d);
        q8[b * qb + l] = (int8_t)q;
        if (ef) {
          const float p = q27o_h2f(dh) * (float)q;
          ef[(size_t)r * n + (size_t)b * qb + l] = y[l] - p;
        }
      }
    }
  }
}

/* add_norm_rows_q8 (src/prefill.cu:372-406): x += (dequant(own) + dequant(recv)) with dequant = fp16 scale * int8
 * (both products exact), then the row norm of add_norm_rows. */
void q27o_add_norm_rows_q8(float* x, const uint8_t* own, const uint8_t* recv, int n, int M, const float* w, float eps,
                           float* h, int8_t* xq, float* xd, float* xs, int qb) {
  const size_t rb = (size_t)n + 2 * (size_t)n / qb;
  for (int r = 0; r < M; r++) {
    float* xr = x + (size_t)r * n;
    const int8_t* oq = (const int8_t*)(own + r * rb);
    const int8_t* rq = (const int8_t*)(recv + r * rb);
    const uint8_t* os = own + r * rb + n;
    const uint8_t* rs = recv + r * rb + n;
    for (int i = 0; i < n; i++) {
      const int b = i / qb;
      const float od = q27o_h2f((uint16_t)(os[2 * b] | (os[2 * b + 1] << 8)));
      const float rd = q27o_h2f((uint16_t)(rs[2 * b] | (rs[2 * b + 1] << 8)));
      const float a = od * (float)oq[i], c = rd * (float)rq[i];
      xr[i] = xr[i] + (a + c);
    }
    norm_q8_row(xr, w, eps, n, (size_t)r, h, xq, xd, xs);
  }
}

/* swiglu_q8 (src/ops.cu:262-270): silu(g) * u -> q8_1 over n values (n % 32 == 0). */
void q27o_swiglu_q8(const float* g, const float* u, int8_t* xq, float* xd, int n, float* xs) {
  float y[32];
  for (int b = 0; b < n / 32; b++) {
    for (int l = 0; l < 32; l++) y[l] = q27o_silu(g[32 * b + l]) * u[32 * b + l];
    q8_block(y, xq, xd, xs, 32 * (size_t)b);
  }
}

/* gated_rmsnorm (src/ops.cu:574-585): block of 128 threads per head of n values. */
void q27o_gated_rmsnorm(const float* o, const float* w, const float* z, float* y, int n, int heads, float eps) {
  float part[1024];
  for (int hd = 0; hd < heads; hd++) {
    const size_t off = (size_t)hd * n;
    thread_sq(o + off, n, 128, part);
    const float t = block_sum(part, 128);
    const float scale = 1.0f / sqrtf(t / (float)n + eps);
    for (int i = 0; i < n; i++) y[off + i] = (scale * o[off + i] * w[i]) * q27o_silu(z[off + i]);
  }
}

/* gated_rmsnorm_q8 (src/ops.cu:272-283): one value per thread, heads of 128. */
void q27o_gated_rmsnorm_q8(const float* o, const float* w, const float* z, int8_t* xq, float* xd, int heads, float eps,
                           float* xs) {
  float part[128], y[128];
  for (int hd = 0; hd < heads; hd++) {
    const size_t off = (size_t)hd * 128;
    for (int i = 0; i < 128; i++) part[i] = o[off + i] * o[off + i];
    const float t = block_sum(part, 128);
    const float scale = 1.0f / sqrtf(t / 128.0f + eps);
    for (int i = 0; i < 128; i++) y[i] = (scale * o[off + i] * w[i]) * q27o_silu(z[off + i]);
    for (int b = 0; b < 4; b++) q8_block(y + 32 * b, xq, xd, xs, off + 32 * (size_t)b);
  }
}

/* l2norm_heads (src/ops.cu:433-447): warp per (token, head); lane sums p[i]^2 for i = lane, lane + 32, ...,
 * then warp_sum; x <- (x * rsqrt(acc/n + eps/n)) * (1/sqrt(n)). */
static void l2_head(float* p, int n, float eps) {
  float a[32];
  for (int l = 0; l < 32; l++) {
    float acc = 0.0f;
    for (int i = l; i < n; i += 32) acc += p[i] * p[i];
    a[l] = acc;
  }
  const float acc = butterfly(a, 32);
  const float scale = 1.0f / sqrtf(acc / (float)n + eps / (float)n);
  const float post = 1.0f / sqrtf((float)n);
  for (int i = 0; i < n; i++) p[i] = (p[i] * scale) * post;
}

void q27o_l2norm_heads(float* x, int n, int heads, int T, int stride, float eps) {
  for (int t = 0; t < T; t++)
    for (int h = 0; h < heads; h++) l2_head(x + (size_t)t * stride + (size_t)h * n, n, eps);
}

/* gdn_gates (src/ops.cu:396-405): beta = sigmoid(b), g = softplus(a + dt_bias) * ssm_a over [T][H]. */
void q27o_gdn_gates(const float* a, const float* b, const float* ssm_a, const float* dt_bias, float* g, float* beta, int H,
                    int T) {
  for (int i = 0; i < H * T; i++) {
    const int h = i % H;
    beta[i] = q27o_sigmoid(b[i]);
    g[i] = q27o_softplus(a[i] + dt_bias[h]) * ssm_a[h];
  }
}

/* 4-tap causal conv of one channel: sum = 0; sum += s0 w0; sum += s1 w1; sum += s2 w2; sum += x w3 (src/ops.cu:419-424) */
static float conv4(float s0, float s1, float s2, float xn, const float* w4) {
  float sum = 0.0f;
  sum += s0 * w4[0];
  sum += s1 * w4[1];
  sum += s2 * w4[2];
  sum += xn * w4[3];
  return sum;
}

/* gdn_conv (src/ops.cu:407-431): planes [4][C][3], oldest tap first. */
void q27o_gdn_conv(const float* x, const float* w, float* planes, int in_plane, float* y, int C, int T, int snapshots) {
  for (int c = 0; c < C; c++) {
    const float* st = planes + ((size_t)in_plane * C + c) * 3;
    float s0 = st[0], s1 = st[1], s2 = st[2];
    for (int t = 0; t < T; t++) {
      const float xn = x[(size_t)t * C + c];
      y[(size_t)t * C + c] = q27o_silu(conv4(s0, s1, s2, xn, w + 4 * (size_t)c));
      s0 = s1; s1 = s2; s2 = xn;
      if (snapshots || t == T - 1) {
        float* o = planes + ((size_t)t * C + c) * 3;
        o[0] = s0; o[1] = s1; o[2] = s2;
      }
    }
  }
}

/* gdn_conv_l2 (src/ops.cu:285-338): gdn_conv, then l2 norm of heads < n_norm_heads (lane order as
 * l2norm_heads), gates of v head (head - n_norm_heads) for tokens 0..T-1. */
void q27o_gdn_conv_l2(const float* x, const float* w, float* planes, int in_plane, float* y, int C, int T, int snapshots,
                      int n_norm_heads, float eps, const float* a, const float* b, const float* ssm_a, const float* dt_bias,
                      float* g, float* beta, int H) {
  q27o_gdn_conv(x, w, planes, in_plane, y, C, T, snapshots);
  q27o_l2norm_heads(y, 128, n_norm_heads, T, C, eps);
  q27o_gdn_gates(a, b, ssm_a, dt_bias, g, beta, H, T);
}

/* gdn_conv_prefill (src/prefill.cu:141-184): per (token t, channel c) the taps are x[t-3..t] with rows < 0 taken
 * from plane in_plane; l2 norm / gates as in gdn_conv_l2; the last 3 inputs go to plane (in_plane == 0 ? 1 : 0). */
void q27o_gdn_conv_prefill(const float* x, const float* w, float* planes, int in_plane, float* y, int C, int M,
                           int n_norm_heads, float eps, const float* a, const float* b, const float* ssm_a,
                           const float* dt_bias, float* g, float* beta, int H) {
  const int out_plane = in_plane == 0 ? 1 : 0;
  for (int c = 0; c < C; c++) {
    const float* st = planes + ((size_t)in_plane * C + c) * 3;
#define Q27_IN(tt) ((tt) >= 0 ? x[(size_t)(tt) * C + c] : st[3 + (tt)])
    for (int t = 0; t < M; t++)
      y[(size_t)t * C + c] = q27o_silu(conv4(Q27_IN(t - 3), Q27_IN(t - 2), Q27_IN(t - 1), x[(size_t)t * C + c], w + 4 * (size_t)c));
    const float o0 = Q27_IN(M - 3), o1 = Q27_IN(M - 2), o2 = Q27_IN(M - 1);
#undef Q27_IN
    float* o = planes + ((size_t)out_plane * C + c) * 3;
    o[0] = o0; o[1] = o1; o[2] = o2;
  }
  q27o_l2norm_heads(y, 128, n_norm_heads, M, C, eps);
  q27o_gdn_gates(a, b, ssm_a, dt_bias, g, beta, H, M);
}

/* kv_cache_bytes (src/attn.cu:890-892): q8_0 = [nkvh][n_ctx][256] int8 + [nkvh][n_ctx][8] fp16; f16 = 2 bytes each. */
size_t q27o_kv_cache_bytes(int nkvh, int n_ctx, int q8) {
  return q8 ? (size_t)nkvh * (size_t)n_ctx * (256 + 16) : (size_t)nkvh * (size_t)n_ctx * 256 * 2;
}

/* attn_prep (src/ops.cu:588-654): per (token, head) RMSNorm over 256 (block of 256 threads) * norm weight;
 * NeoX rotation of pairs (j, j + 32), j < 32, theta = p * theta_scale^j with p = rope3[t][j % 3] (IMRoPE) or
 * pos0 + t - rdelta; q -> qn [T][nqh][256]; k (rotated) and v -> cache row kh * n_ctx + pos0 + t as f16, or
 * q8_0 (d = amax/127, q = roundf(x * (d ? 1/d : 0)), fp16 scales after the int8 area). Rows outside
 * [0, n_ctx) are not written. */
void q27o_attn_prep(const float* qg, const float* k, const float* v, const float* q_norm, const float* k_norm, float* qn,
                    void* kcache, void* vcache, int pos0, int T, float eps, float theta_scale, int nqh, int nkvh, int n_ctx,
                    int q8, const int* rope3, const int* rdelta) {
  float freq[32];
  q27o_rope_freqs(theta_scale, freq);
  for (int tok = 0; tok < T; tok++) {
    const int pos = pos0 + tok;
    for (int hb = 0; hb < nqh + nkvh; hb++) {
      const int isq = hb < nqh;
      const float* src = isq ? qg + (size_t)tok * nqh * 512 + (size_t)hb * 512 : k + ((size_t)tok * nkvh + (hb - nqh)) * 256;
      const float* w = isq ? q_norm : k_norm;
      float part[256], buf[256], out[256];
      for (int d = 0; d < 256; d++) part[d] = src[d] * src[d];
      const float t = block_sum(part, 256);
      const float scale = 1.0f / sqrtf(t / 256.0f + eps);
      for (int d = 0; d < 256; d++) buf[d] = scale * src[d] * w[d];
      for (int d = 0; d < 256; d++) {
        out[d] = buf[d];
        if (d < 64) {
          const int j = d & 31;
          const int rp = rope3 ? rope3[tok * 3 + j % 3] : pos - (rdelta ? *rdelta : 0);
          const float theta = (float)rp * freq[j];
          float sn, cs;
          q27o_sincos(theta, &sn, &cs);
          const float x0 = buf[j], x1 = buf[j + 32];
          out[d] = d < 32 ? x0 * cs - x1 * sn : x0 * sn + x1 * cs;
        }
      }
      if (isq) {
        memcpy(qn + ((size_t)tok * nqh + hb) * 256, out, sizeof out);
        continue;
      }
      if (pos < 0 || pos >= n_ctx) continue;
      const int kh = hb - nqh;
      const size_t row = (size_t)kh * n_ctx + pos;
      const float* vv = v + ((size_t)tok * nkvh + kh) * 256;
      if (!q8) {
        uint16_t* kc = (uint16_t*)kcache;
        uint16_t* vc = (uint16_t*)vcache;
        for (int d = 0; d < 256; d++) {
          kc[row * 256 + d] = q27o_f2h(out[d]);
          vc[row * 256 + d] = q27o_f2h(vv[d]);
        }
      } else {
        const size_t so = (size_t)nkvh * n_ctx * 256;
        int8_t* kq = (int8_t*)kcache;
        int8_t* vq = (int8_t*)vcache;
        uint16_t* ks = (uint16_t*)((uint8_t*)kcache + so);
        uint16_t* vs = (uint16_t*)((uint8_t*)vcache + so);
        for (int b = 0; b < 8; b++) {
          float ak = 0.0f, av = 0.0f;
          for (int l = 0; l < 32; l++) {
            ak = fmaxf(ak, fabsf(out[32 * b + l]));
            av = fmaxf(av, fabsf(vv[32 * b + l]));
          }
          const float dk = ak / 127.f, dv = av / 127.f;
          const float ik = dk != 0.0f ? 1.0f / dk : 0.0f, iv = dv != 0.0f ? 1.0f / dv : 0.0f;
          for (int l = 0; l < 32; l++) {
            kq[row * 256 + 32 * b + l] = (int8_t)roundf(out[32 * b + l] * ik);
            vq[row * 256 + 32 * b + l] = (int8_t)roundf(vv[32 * b + l] * iv);
          }
          ks[row * 8 + b] = q27o_f2h(dk);
          vs[row * 8 + b] = q27o_f2h(dv);
        }
      }
    }
  }
}

/* ------------------------------------------------------------------------------------------------ gathers */
static const uint64_t iq2s_grid_tab[1024] = {
#include "../qwen27-engine_amd/csrc/iq2s_grid.inc"
};
const uint64_t* q27o_iq2s_grid(void) { return iq2s_grid_tab; }

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* An id < 0 selects row (-id - 1) of img (src/ops.cu:352-358); with img null such a row is written as zeros. */
static int img_row(int id, float* out, int n, const float* img) {
  if (id >= 0) return 0;
  for (int i = 0; i < n; i++) out[i] = img ? img[(size_t)(-id - 1) * n + i] : 0.0f;
  return 1;
}

/* get_rows_iq2_s (src/ops.cu:340-375), ggml dequantize_row_iq2_s order: 82-byte block = d (f16), qs[32],
 * signs[32], qh[8], scales[8]; group ib32 of 32 weights, 4 sub-groups l of 8:
 * db = d * (0.5 + (l < 2 ? sc & 15 : sc >> 4)) * 0.25, y = db * grid * sign. */
void q27o_get_rows_iq2_s(const uint8_t* table, int64_t row_bytes, const int* ids, int T, float* y, int n, const float* img) {
  for (int tok = 0; tok < T; tok++) {
    float* out = y + (size_t)tok * n;
    if (img_row(ids[tok], out, n, img)) continue;
    const uint8_t* rowp = table + (size_t)ids[tok] * (size_t)row_bytes;
    for (int sb = 0; sb < n / 256; sb++) {
      const uint8_t* b = rowp + (size_t)sb * 82;
      const float d = q27o_h2f(rd16(b));
      for (int ib32 = 0; ib32 < 8; ib32++) {
        const uint8_t qh = b[66 + ib32], sc = b[74 + ib32];
        for (int l = 0; l < 4; l++) {
          const float db = d * (0.5f + (float)((l < 2 ? sc : sc >> 4) & 0xF)) * 0.25f;
          const uint64_t gv = iq2s_grid_tab[b[2 + 4 * ib32 + l] | ((qh << (8 - 2 * l)) & 0x300)];
          const uint8_t sg = b[34 + 4 * ib32 + l];
          for (int j = 0; j < 8; j++) {
            const float gval = (float)((gv >> (8 * j)) & 0xFF);
            out[sb * 256 + 32 * ib32 + 8 * l + j] = db * gval * ((sg >> j) & 1 ? -1.f : 1.f);
          }
        }
      }
    }
  }
}

/* Q4_K (ggml dequantize_row_q4_K; transcribed order src/requant.cpp:90-114): 144-byte block = d, dmin (f16),
 * scales[12] (6-bit scale/min pairs, get_scale_min_k4), qs[128]; y = (d * sc) * q - (dmin * m). */
static void scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m) {
  if (j < 4) {
    *d = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
    *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
  }
}

void q27o_get_rows_q4_k(const uint8_t* table, int64_t row_bytes, const int* ids, int T, float* y, int n, const float* img) {
  for (int tok = 0; tok < T; tok++) {
    float* out = y + (size_t)tok * n;
    if (img_row(ids[tok], out, n, img)) continue;
    const uint8_t* rowp = table + (size_t)ids[tok] * (size_t)row_bytes;
    for (int sb = 0; sb < n / 256; sb++) {
      const uint8_t* b = rowp + (size_t)sb * 144;
      const float d = q27o_h2f(rd16(b)), mn = q27o_h2f(rd16(b + 2));
      const uint8_t* q = b + 16;
      float* yo = out + sb * 256;
      for (int j = 0; j < 4; j++) {
        uint8_t sc, m;
        scale_min_k4(2 * j, b + 4, &sc, &m);
        const float d1 = d * (float)sc, m1 = mn * (float)m;
        scale_min_k4(2 * j + 1, b + 4, &sc, &m);
        const float d2 = d * (float)sc, m2 = mn * (float)m;
        for (int l = 0; l < 32; l++) yo[64 * j + l] = d1 * (float)(q[32 * j + l] & 0xF) - m1;
        for (int l = 0; l < 32; l++) yo[64 * j + 32 + l] = d2 * (float)(q[32 * j + l] >> 4) - m2;
      }
    }
  }
}

/* Q6_K (ggml dequantize_row_q6_K; transcribed order src/requant.cpp:68-88): 210-byte block = ql[128], qh[64],
 * scales[16] (int8), d (f16); y = (d * sc) * (q6 - 32). */
void q27o_get_rows_q6_k(const uint8_t* table, int64_t row_bytes, const int* ids, int T, float* y, int n, const float* img) {
  for (int tok = 0; tok < T; tok++) {
    float* out = y + (size_t)tok * n;
    if (img_row(ids[tok], out, n, img)) continue;
    const uint8_t* rowp = table + (size_t)ids[tok] * (size_t)row_bytes;
    for (int sb = 0; sb < n / 256; sb++) {
      const uint8_t* b = rowp + (size_t)sb * 210;
      const float d = q27o_h2f(rd16(b + 208));
      for (int half = 0; half < 2; half++) {
        const uint8_t* ql = b + 64 * half;
        const uint8_t* qh = b + 128 + 32 * half;
        const int8_t* sc = (const int8_t*)(b + 192 + 8 * half);
        float* yo = out + sb * 256 + 128 * half;
        for (int l = 0; l < 32; l++) {
          const int is = l / 16;
          const int q1 = ((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
          const int q2 = ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
          const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
          const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
          yo[l] = d * (float)sc[is] * (float)q1;
          yo[l + 32] = d * (float)sc[is + 2] * (float)q2;
          yo[l + 64] = d * (float)sc[is + 4] * (float)q3;
          yo[l + 96] = d * (float)sc[is + 6] * (float)q4;
        }
      }
    }
  }
}

/* Q8_0 (ggml block_q8_0 / dequantize_row_q8_0): 34-byte block = d (f16), qs[32] int8; y = q * d. */
void q27o_get_rows_q8_0(const uint8_t* table, int64_t row_bytes, const int* ids, int T, float* y, int n, const float* img) {
  for (int tok = 0; tok < T; tok++) {
    float* out = y + (size_t)tok * n;
    if (img_row(ids[tok], out, n, img)) continue;
    const uint8_t* rowp = table + (size_t)ids[tok] * (size_t)row_bytes;
    for (int blk = 0; blk < n / 32; blk++) {
      const uint8_t* b = rowp + (size_t)blk * 34;
      const float d = q27o_h2f(rd16(b));
      for (int l = 0; l < 32; l++) out[32 * blk + l] = (float)(int8_t)b[2 + l] * d;
    }
  }
}
