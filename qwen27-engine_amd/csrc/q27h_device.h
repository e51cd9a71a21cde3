// Device helpers shared by the gfx950 kernels of the fused per-layer ops.
//
// Numerics contract (identical on the CPU checker): no FP contraction (built with -ffp-contract=off),
// rsqrt = 1.0f / sqrtf, correctly rounded division and sqrt, exp/log/sin/cos from the routines below.
// Lane exchanges use DPP (quad permutes, 16-lane row rotates), v_permlane16_swap (xor 16) and ds_swizzle /
// ds_bpermute for the remaining patterns; they only move values, so every reduction below adds exactly the operands the reference's 32-lane
// butterflies add (src/ops.cu:34-50, src/common.cuh:68-87).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace q27h {

constexpr int kRowN = 5120;  // hidden size of the row kernels (n must be 5120, src/ops.cu:699)
constexpr int kCUs = 256;    // compute units of an MI355X (8 XCDs of 32), the grid unit of the persistent kernels

// ---------------------------------------------------------------- lane exchange
// Value of lane (lane ^ M), M in {1, 2, 4, 7, 8, 16, 24}: stays inside an aligned group of 32 lanes.
template <int M>
__device__ __forceinline__ float lane_xor(float v) {
  const int iv = __builtin_bit_cast(int, v);
  int r;
  // bound_ctrl set: every source lane of these patterns is in range, and the backend can then fold the move into
  // the consuming add / max as a DPP operand (one instruction instead of two)
  if constexpr (M == 1) r = __builtin_amdgcn_mov_dpp(iv, 0xB1, 0xF, 0xF, true);        // quad_perm [1,0,3,2]
  else if constexpr (M == 2) r = __builtin_amdgcn_mov_dpp(iv, 0x4E, 0xF, 0xF, true);   // quad_perm [2,3,0,1]
  else if constexpr (M == 8) r = __builtin_amdgcn_mov_dpp(iv, 0x128, 0xF, 0xF, true);  // row_ror:8 (16-lane rows)
  else if constexpr (M == 7) r = __builtin_amdgcn_mov_dpp(iv, 0x141, 0xF, 0xF, true);  // row_half_mirror: l ^ 7 in 8
  else if constexpr (M == 16) {
    // v_permlane16_swap of a value with itself: the first result holds row 0 in rows 0 and 1 (row 2 in rows 2 and 3),
    // the second row 1 in rows 0 and 1 (row 3 in rows 2 and 3), so the partner row of lane l is the second result
    // for l & 16 == 0 and the first otherwise (a VALU exchange, no LDS round trip)
    const auto pr = __builtin_amdgcn_permlane16_swap(iv, iv, false, false);
    r = (__lane_id() & 16) ? (int)pr[0] : (int)pr[1];
  } else r = __builtin_amdgcn_ds_swizzle(iv, (M << 10) | 0x1F);                        // bit mode: lane ^ M
  return __builtin_bit_cast(float, r);
}
// Value of lane ((lane & AND) | OR) inside the same 32-lane group (ds_swizzle bit mode).
template <int AND, int OR>
__device__ __forceinline__ float lane_pick(float v) {
  const int iv = __builtin_bit_cast(int, v);
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(iv, (OR << 5) | AND));
}
// Value of lane (lane ^ 32): crosses the two halves of the wave (v_permlane32_swap, then the half's own copy).
__device__ __forceinline__ float lane_xor32(float v) {
  const int iv = __builtin_bit_cast(int, v);
  const auto pr = __builtin_amdgcn_permlane32_swap(iv, iv, false, false);
  return __builtin_bit_cast(float, (__lane_id() & 32) ? (int)pr[0] : (int)pr[1]);
}

// ---------------------------------------------------------------- scheduling
// Ends a block of loads: the compiler may not move any instruction across it, so every load above is issued
// before the first use of any of them (otherwise the scheduler hoists a use of the first value between the loads and
// the waitcnt it needs holds back the remaining loads by a full memory round trip).
__device__ __forceinline__ void loads_issued() { __builtin_amdgcn_sched_barrier(0); }
// Makes the listed kernel arguments live in SGPRs at this point. Placed at kernel entry it turns the compiler's
// deferred kernarg loads (each a dependent round trip to the kernarg buffer after the launch's cache invalidation)
// into one batch of scalar loads issued together.
template <typename T>
__device__ __forceinline__ void arg_now(T a) {
  asm volatile("" ::"s"(a));
}
template <typename... A>
__device__ __forceinline__ void args_now(A... a) {
  (arg_now(a), ...);
}

// ---------------------------------------------------------------- lane layout of a 32-value block
// Eight lanes hold one block of 32 consecutive values, four per lane. Lane q (= lane & 7) holds the four values at
// 4 * quad_of_lane(q): lanes 0..3 take quads 0..3 and lanes 4..7 quads 7..4. With this order the reference's
// butterfly over the block's 32 virtual lanes (xor 16, 8, 4, 2, 1) is lane xor 7 (row_half_mirror), lane xor 2,
// lane xor 1 (quad permutes) and then the lane's own value pairs: DPP operands that fold into the adds. The loads
// and stores of the 8 lanes still cover the block's 128 bytes exactly.
__device__ __forceinline__ int quad_of_lane(int q) { return q < 4 ? q : 11 - q; }
// Offset (in values) of this thread's four values inside its group's 32-value block.
__device__ __forceinline__ int block_offset(int lane) { return 4 * quad_of_lane(lane & 7); }

// The reference's warp_sum (xor 16, 8, 4, 2, 1 over the 32 lanes of a lane group).
__device__ __forceinline__ float warp32_sum(float v) {
  v += lane_xor<16>(v);
  v += lane_xor<8>(v);
  v += lane_xor<4>(v);
  v += lane_xor<2>(v);
  v += lane_xor<1>(v);
  return v;
}

// Reference block_sum (src/ops.cu:40-50) for a block of `nthreads` threads (multiple of 32), one value per
// thread, thread t = threadIdx.x. `red` is 32 floats of LDS. All threads must call it.
__device__ __forceinline__ float block_sum_ref(float v, float* red, int nthreads) {
  const int t = threadIdx.x;
  v = warp32_sum(v);
  __syncthreads();
  if ((t & 31) == 0) red[t >> 5] = v;
  __syncthreads();
  v = (t & 31) < (nthreads >> 5) ? red[t & 31] : 0.0f;
  return warp32_sum(v);
}

// ---------------------------------------------------------------- conversions
__device__ __forceinline__ uint16_t f2h_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);  // v_cvt_f16_f32: round to nearest even, subnormals kept
}
__device__ __forceinline__ float h2f_bits(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ float fp16_round(float f) { return (float)(_Float16)f; }
// __float2bfloat16 (round to nearest even; NaN stays a quiet NaN)
__device__ __forceinline__ float bf16_round(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return __builtin_bit_cast(float, (u | 0x00400000u) & 0xffff0000u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return __builtin_bit_cast(float, u & 0xffff0000u);
}
__device__ __forceinline__ float bf16_to_f(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }

// ---------------------------------------------------------------- global loads and stores
__device__ __forceinline__ float4 ld4(const float* p) { return *(const float4*)p; }
// 16-byte streaming load (nontemporal hint: the data is read once), used where it measured faster: the SwiGLU
// and quantizer inputs, the gated-norm inputs and the attention q/k/v.
typedef float q27_v4f __attribute__((ext_vector_type(4)));
#ifndef Q27H_NT
#define Q27H_NT 1
#endif
__device__ __forceinline__ float4 ld4_nt(const float* p) {
#if Q27H_NT
  const q27_v4f v = __builtin_nontemporal_load((const q27_v4f*)p);
  return make_float4(v.x, v.y, v.z, v.w);
#else
  return *(const float4*)p;
#endif
}
// Stores. NT = nontemporal (streaming) hint, chosen per kernel from measurement: it pays where the written data
// would otherwise still be draining from the caches when the next kernel runs.
template <bool NT = false>
__device__ __forceinline__ void st4(float* p, float a, float b, float c, float d) {
  if constexpr (NT) {
    const q27_v4f v = {a, b, c, d};
    __builtin_nontemporal_store(v, (q27_v4f*)p);
  } else {
    *(float4*)p = make_float4(a, b, c, d);
  }
}
template <bool NT = false>
__device__ __forceinline__ void st_u32(void* p, uint32_t v) {
  if constexpr (NT) __builtin_nontemporal_store(v, (uint32_t*)p);
  else *(uint32_t*)p = v;
}
template <bool NT = false>
__device__ __forceinline__ void st_f32(float* p, float v) {
  if constexpr (NT) __builtin_nontemporal_store(v, p);
  else *p = v;
}

// ---------------------------------------------------------------- transcendental functions
// exp: Cody-Waite reduction x = k ln2 + r, degree-7 Taylor polynomial of e^r (Horner, fma), ldexp.
// Same operations and constants as the CPU checker (Muller, Elementary Functions, ch. 11).
// The reduction, polynomial and scaling of q27_expf, valid where no clamp or special case applies (|x| <= 87).
__device__ __forceinline__ float q27_expf_core(float x) {
  const float k = __builtin_rintf(x * 1.44269502f);
  float r = __builtin_fmaf(-k, 0.693145752f, x);
  r = __builtin_fmaf(-k, 1.42860677e-06f, r);
  float p = 1.98412698e-4f;
  p = __builtin_fmaf(p, r, 1.38888889e-3f);
  p = __builtin_fmaf(p, r, 8.33333333e-3f);
  p = __builtin_fmaf(p, r, 4.16666667e-2f);
  p = __builtin_fmaf(p, r, 1.66666667e-1f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  return __builtin_ldexpf(p, (int)k);
}

__device__ __forceinline__ float q27_expf(float x) {
  // Branch-free: the polynomial is evaluated on a clamped argument and the out-of-range results are selected
  // afterwards, giving the same values as the early-return form of the CPU checker.
  const float xc = __builtin_fminf(__builtin_fmaxf(x, -103.972084f), 88.7228394f);
  float e = q27_expf_core(xc);
  e = x > 88.7228394f ? __builtin_huge_valf() : e;
  e = x < -103.972084f ? 0.0f : e;
  return x != x ? x + x : e;
}

// x / d for silu's operands, correctly rounded: d = 1 + q27_expf_core(-x) with 2^-60 <= |x| <= 60. The steps of gfx9's
// IEEE division sequence (reciprocal, one Newton step, quotient, residual correction) without its range scaling and
// fix-up, which leave every operand unchanged here, and with one residual correction instead of two: over every
// float x of that range (3.3e9 cases with the hardware reciprocal modelled as the correctly rounded one moved by -1, 0
// or +1 ulp; tests/test_device_silu_div.py) the one-correction quotient equals the two-correction one and x / d. The
// single exception, shared by both sequences, is x = 2^-23 (d = 2 - 2^-23) with a reciprocal one ulp off; the GPU
// test of silu covers that argument on the hardware.
__device__ __forceinline__ float div_silu(float x, float d) {
  const float y0 = __builtin_amdgcn_rcpf(d);
  const float e = __builtin_fmaf(-d, y0, 1.0f);
  const float y = __builtin_fmaf(e, y0, y0);
  const float q0 = x * y;
  const float r0 = __builtin_fmaf(-d, q0, x);
  return __builtin_fmaf(r0, y, q0);
}

// log for the softplus gate: x = 2^e m, m in [sqrt(1/2), sqrt(2)), s = f / (2 + f), log m = 2 atanh(s) as an
// odd series to s^11, log x = e ln2_hi + (e ln2_lo + log m).
__device__ __forceinline__ float q27_logf(float x) {
  if (x != x || x < 0.0f) return __builtin_nanf("");
  if (x == 0.0f) return -__builtin_huge_valf();
  if (x == __builtin_huge_valf()) return x;
  int e = 0;
  if (x < 1.17549435e-38f) { x *= 8388608.0f; e = -23; }
  uint32_t ix = __builtin_bit_cast(uint32_t, x);
  e += (int)((ix >> 23) & 0xff) - 127;
  ix = (ix & 0x007fffffu) | 0x3f800000u;
  float m = __builtin_bit_cast(float, ix);
  if (m > 1.41421354f) { m *= 0.5f; e += 1; }
  const float f = m - 1.0f;
  const float s = f / (2.0f + f);
  const float z = s * s;
  float R = 1.81818187e-1f;
  R = __builtin_fmaf(R, z, 2.22222224e-1f);
  R = __builtin_fmaf(R, z, 2.85714298e-1f);
  R = __builtin_fmaf(R, z, 4.00000006e-1f);
  R = __builtin_fmaf(R, z, 6.66666687e-1f);
  R = R * z;
  const float logm = __builtin_fmaf(s, R, s + s);
  const float fe = (float)e;
  return __builtin_fmaf(fe, 0.693145752f, __builtin_fmaf(fe, 1.42860677e-06f, logm));
}

// silu(x) = x / (1 + e^-x). For 2^-60 <= |x| <= 60 the exp needs no clamp and the division is div_silu's
// (1 + e^-x <= 2^87); other arguments (zeros, subnormals, large or non-finite values) take the general path.
__device__ __forceinline__ float q27_silu(float x) { return x / (1.0f + q27_expf(-x)); }
__device__ __forceinline__ bool silu_fast_ok(float x) {
  const float ax = __builtin_fabsf(x);
  return ax >= 0x1p-60f && ax <= 60.0f;
}
// silu on the fast range only (2^-60 <= |x| <= 60, see silu_fast_ok); equal to q27_silu there.
__device__ __forceinline__ float silu_fast(float x) { return div_silu(x, 1.0f + q27_expf_core(-x)); }
// N values at once, one branch for the lanes with an argument outside the fast range.
template <int N>
__device__ __forceinline__ void q27_silu_n(const float (&x)[N], float (&out)[N]) {
  bool ok = true;
#pragma unroll
  for (int k = 0; k < N; k++) {
    out[k] = div_silu(x[k], 1.0f + q27_expf_core(-x[k]));
    ok &= silu_fast_ok(x[k]);
  }
  if (!ok) {
#pragma unroll
    for (int k = 0; k < N; k++) out[k] = q27_silu(x[k]);
  }
}
// silu within a few float32 ulps (not bit-exact): x * sigmoid(x) from e = 2^(-|x| log2 e) in (0, 1] on the hardware
// exp2 (the product's rounding restored by one first-order term), the hardware reciprocal of 1 + e with one Newton
// step, and x * e / (1 + e) for negative x. No overflow anywhere: e <= 1 and 1 <= 1 + e <= 2. Relative error below
// 1e-6 for |x| <= 87; for x < -87 the value is a tiny negative number where the correctly rounded quotient
// x / (1 + e^-x) is -0 or subnormal.
__device__ __forceinline__ float silu_tol(float x) {
  const float ax = __builtin_fabsf(x);
  const float t = ax * -1.44269502f;
  const float lo = __builtin_fmaf(ax, -1.44269502f, -t) + ax * -1.925963e-8f;  // -|x| log2 e - t
  float e = __builtin_amdgcn_exp2f(t);
  e = __builtin_fmaf(e, lo * 0.693147181f, e);
  const float d = 1.0f + e;
  float r = __builtin_amdgcn_rcpf(d);
  r = __builtin_fmaf(__builtin_fmaf(-d, r, 1.0f), r, r);
  return x * (x < 0.0f ? e * r : r);
}
// Q27H_SILU_LEAN = 1 (the default): the tolerance SiLU is silu_lean below, not silu_tol. Measured in
// gdn_conv_prefill (M = 2048, three alternating rounds on one box, with the L2 scale on the hardware rsq beside it):
// 34.8-35.4 against 35.9-36.2 us per launch, and 10.365-10.378 against 10.365-10.438 ms per prefill pass.
#ifndef Q27H_SILU_LEAN
#define Q27H_SILU_LEAN 1
#endif
// silu_tol without the product's rounding term and the Newton step: e = 2^(-|x| log2 e) on the hardware exp2 (the
// argument's rounding moves e by up to |x| 2^-24 relative), the hardware reciprocal of 1 + e. Relative error below
// 4.1e-6 on [-87, 87] with both hardware operations off by one ulp (the fp32 tolerance of the path is 1e-5); the error
// profile of an exp2-based expf and an approximate reciprocal, as a fast-math build of the reference computes silu.
__device__ __forceinline__ float silu_lean(float x) {
  const float e = __builtin_amdgcn_exp2f(__builtin_fabsf(x) * -1.44269502f);
  const float r = __builtin_amdgcn_rcpf(1.0f + e);
  return x * (x < 0.0f ? e * r : r);
}
template <int N>
__device__ __forceinline__ void q27_silu_tol_n(const float (&x)[N], float (&out)[N]) {
#pragma unroll
  for (int k = 0; k < N; k++) out[k] = Q27H_SILU_LEAN ? silu_lean(x[k]) : silu_tol(x[k]);
}
__device__ __forceinline__ float q27_sigmoid(float x) { return 1.0f / (1.0f + q27_expf(-x)); }
__device__ __forceinline__ float q27_softplus(float x) { return x > 20.0f ? x : q27_logf(1.0f + q27_expf(x)); }

// sin and cos of a float angle: Cody-Waite reduction by pi/2 in double (pio2 split 33 + 53 bits), Taylor
// polynomials to degree 21 / 20 on |r| <= pi/4, separate double multiplies and adds, one rounding to float.
__device__ __forceinline__ void q27_sincos(float theta, float* s_out, float* c_out) {
  const double th = (double)theta;
  const double kd = __builtin_rint(th * 6.36619772367581382433e-01);
  const double r = (th - kd * 1.57079632673412561417e+00) - kd * 6.07710050650619224932e-11;
  const double z = r * r;
  double sp = 1.9572941063391263e-20;
  sp = sp * z + -8.22063524662433e-18;
  sp = sp * z + 2.8114572543455206e-15;
  sp = sp * z + -7.647163731819816e-13;
  sp = sp * z + 1.6059043836821613e-10;
  sp = sp * z + -2.505210838544172e-08;
  sp = sp * z + 2.7557319223985893e-06;
  sp = sp * z + -0.0001984126984126984;
  sp = sp * z + 0.008333333333333333;
  sp = sp * z + -0.16666666666666666;
  const double sn = r + (r * z) * sp;
  double cp = 4.110317623312165e-19;
  cp = cp * z + -1.5619206968586225e-16;
  cp = cp * z + 4.779477332387385e-14;
  cp = cp * z + -1.1470745597729725e-11;
  cp = cp * z + 2.08767569878681e-09;
  cp = cp * z + -2.755731922398589e-07;
  cp = cp * z + 2.48015873015873e-05;
  cp = cp * z + -0.001388888888888889;
  cp = cp * z + 0.041666666666666664;
  cp = cp * z + -0.5;
  const double cs = 1.0 + z * cp;
  const int q = (int)(long long)kd & 3;
  double s, c;
  if (q == 0) { s = sn; c = cs; }
  else if (q == 1) { s = cs; c = -sn; }
  else if (q == 2) { s = -sn; c = -cs; }
  else { s = -cs; c = sn; }
  *s_out = (float)s;
  *c_out = (float)c;
}

// ---------------------------------------------------------------- q8 rounding
// amax / 127, correctly rounded, for amax >= 0: q0 = amax * RN(1/127), then one residual correction
// r = amax - 127 q0 (exact in an fma), q0 + r * RN(1/127). The result equals the IEEE quotient for every finite
// amax >= 0, subnormals included (checked exhaustively over all 2^31 non-negative finite floats on the host);
// amax = +inf gives +inf and NaN stays NaN.
constexpr float kInv127 = 1.0f / 127.0f;
__device__ __forceinline__ float div127(float amax) {
  const float q0 = amax * kInv127;
  const float r = __builtin_fmaf(-127.0f, q0, amax);
  const float q1 = __builtin_fmaf(r, kInv127, q0);
  return amax == __builtin_huge_valf() ? amax : q1;
}

// roundf(y / d) (q = 0 when d == 0) for |y| <= 127 d, branch-free: the quotient is formed with the steps of the IEEE
// division sequence (reciprocal refined by one fma step, two fma residual corrections), which give the correctly
// rounded quotient unless the sequence would have to pre-scale its operands. For 2^-100 <= d <= 2^100 and
// |y / d| >= 1/2 it never would, and a smaller quotient rounds to 0 either way; the result is then rounded half away
// from zero (|y / d| <= 127 (1 + 2^-22) here). Returns false for any other d except 0 (subnormal, tiny, huge, infinite or NaN scales: the caller then
// takes the IEEE quotient).
template <int N>
__device__ __forceinline__ bool q8_quot_exact(const float (&y)[N], float d, int (&q)[N]) {
  const float r = __builtin_amdgcn_rcpf(d);
  // d == 0 (then every y is +-0): a zero reciprocal makes every step below exactly +-0, so q = 0 without a select
  const float r1 = d == 0.0f ? 0.0f : __builtin_fmaf(__builtin_fmaf(-d, r, 1.0f), r, r);
#pragma unroll
  for (int c = 0; c < N; c++) {
    const float q0 = y[c] * r1;
    const float q1 = __builtin_fmaf(__builtin_fmaf(-d, q0, y[c]), r1, q0);
    const float q2 = __builtin_fmaf(__builtin_fmaf(-d, q1, y[c]), r1, q1);
    // roundf(q2) for |q2| <= 130 (checked against roundf for every float in that range): q2 + copysign(0.5 - 2^-25)
    // rounds to nearest, then the conversion truncates
    q[c] = (int)(q2 + __builtin_copysignf(0x1.fffffep-2f, q2));
  }
  return (d == 0.0f) | ((d >= 0x1p-100f) & (d <= 0x1p100f));
}

// roundf(y / d) for |y| <= 127 d (the q8_1 rule of src/common.cuh:76; q = 0 when d == 0), four values at a time.
// For 2^-126 <= d <= 2^126, a = y * rcp(d) (v_rcp_f32 within 1 ulp, then one rounding) is within
// 127 (2^-23 + 2^-24) < 2.3e-5 of the exact quotient y / d, and the correctly rounded quotient within 2^-18 (half an ulp
// below 128) of it; so unless a lies within 2.7e-5 of a half-integer, a and the IEEE quotient round to the same
// integer, and rintf == roundf there. The guard band is 2^-14 = 6.1e-5 (2^-12 measured 40 us per prefill pass slower:
// a wave takes the branch when any of its values falls in the band). Values near a half-integer, NaN, d == 0 and d outside that range take the IEEE quotient:
// one branch per four values, almost never taken.
__device__ __forceinline__ void q8_round_div4(const float (&y)[4], float d, int (&q)[4]) {
  const float rd = __builtin_amdgcn_rcpf(d);
  bool slow = !(d >= 0x1p-126f && d <= 0x1p126f);
#pragma unroll
  for (int c = 0; c < 4; c++) {
    const float a = y[c] * rd;
    const float r = __builtin_rintf(a);
    slow |= !(__builtin_fabsf(a - r) < 0.5f - 0x1p-14f);
    q[c] = (int)r;
  }
  if (slow) {
#pragma unroll
    for (int c = 0; c < 4; c++) q[c] = d == 0.0f ? 0 : (int)__builtin_roundf(y[c] / d);
  }
}

__device__ __forceinline__ uint32_t pack4_i8(int a, int b, int c, int d) {
  return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) | ((uint32_t)(d & 0xff) << 24);
}

// q8_1 of K 32-value blocks held by the 8 lanes of a group in the block layout above: the lane's values of block k
// are the flat indices i0 + k * stride .. + 3 of the arrays xq (values), xd (one scale per 32) and xs (one sum per 16),
// which the caller offsets to a 32-aligned base so that the indices stay 32-bit; blocks k >= kn are not stored (kn
// uniform per 8-lane group). Per block: amax, d = amax / 127, q = roundf(y / d) (0 when amax == 0), xd = fp16(d) as
// f32, and the optional per-16 sums of the unquantized values in the reference's butterfly order (xor 8, 4, 2, 1 over
// the 16 virtual lanes = lane xor 2, lane xor 1, then value pairs (0,2)(1,3), then (0,1)); the block's first 16
// values sit in lanes 0..3 of the group and the last 16 in lanes 4..7. The K dependent chains are formed side by side
// and each kind of store is one guarded group. EXACT: the quotients by q8_quot_exact (branch-free, a few more
// operations per value: for latency-bound launches, where a wave would otherwise often wait on a fallback); else
// q8_round_div4 (fewest operations on average: for throughput-bound launches).
template <bool NT, int K, bool EXACT>
__device__ __forceinline__ void q8_1_store_n(const float (&y)[K][4], int8_t* __restrict__ xq, float* __restrict__ xd,
                                             float* __restrict__ xs, int i0, int stride, int kn = K) {
  float d[K];
#pragma unroll
  for (int k = 0; k < K; k++) {
    float amax = __builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(y[k][0]), __builtin_fabsf(y[k][1])),
                                 __builtin_fmaxf(__builtin_fabsf(y[k][2]), __builtin_fabsf(y[k][3])));
    amax = __builtin_fmaxf(amax, lane_xor<7>(amax));
    amax = __builtin_fmaxf(amax, lane_xor<2>(amax));
    amax = __builtin_fmaxf(amax, lane_xor<1>(amax));
    d[k] = div127(amax);
  }
  int q[K][4];
  if constexpr (EXACT) {
    bool ok = true;
#pragma unroll
    for (int k = 0; k < K; k++) ok &= q8_quot_exact<4>(y[k], d[k], q[k]);
    if (__builtin_expect(__any(!ok), 0)) {  // a scale outside [2^-100, 2^100]: practically never
#pragma unroll
      for (int k = 0; k < K; k++) {
#pragma unroll
        for (int c = 0; c < 4; c++) q[k][c] = d[k] == 0.0f ? 0 : (int)__builtin_roundf(y[k][c] / d[k]);
      }
    }
  } else {
#pragma unroll
    for (int k = 0; k < K; k++) q8_round_div4(y[k], d[k], q[k]);
  }
  float tot[K];
  if (xs) {
#pragma unroll
    for (int k = 0; k < K; k++) {
      float u[4];
#pragma unroll
      for (int c = 0; c < 4; c++) u[c] = y[k][c] + lane_xor<2>(y[k][c]);
#pragma unroll
      for (int c = 0; c < 4; c++) u[c] = u[c] + lane_xor<1>(u[c]);
      tot[k] = (u[0] + u[2]) + (u[1] + u[3]);
    }
  }
#pragma unroll
  for (int k = 0; k < K; k++)
    if (k < kn) st_u32<NT>(xq + i0 + k * stride, pack4_i8(q[k][0], q[k][1], q[k][2], q[k][3]));
  if ((i0 & 31) == 0) {
#pragma unroll
    for (int k = 0; k < K; k++)
      if (k < kn) st_f32<NT>(xd + ((i0 + k * stride) >> 5), fp16_round(d[k]));
  }
  if (xs && (i0 & 15) == 0) {
#pragma unroll
    for (int k = 0; k < K; k++)
      if (k < kn) st_f32<NT>(xs + ((i0 + k * stride) >> 4), tot[k]);
  }
}

// First stage of the reference block_sum for a 32-thread virtual warp held by 8 lanes in the block layout above
// (lane q holds virtual lanes 4 quad_of_lane(q) + c): virtual xor 16, 8, 4 are lane xor 7, 2, 1, and virtual xor 2
// and 1 pair the lane's own values. Every lane of the group returns the virtual warp's sum.
__device__ __forceinline__ float vwarp_sum4(float (&s)[4]) {
#pragma unroll
  for (int c = 0; c < 4; c++) s[c] += lane_xor<7>(s[c]);
#pragma unroll
  for (int c = 0; c < 4; c++) s[c] += lane_xor<2>(s[c]);
#pragma unroll
  for (int c = 0; c < 4; c++) s[c] += lane_xor<1>(s[c]);
  return (s[0] + s[2]) + (s[1] + s[3]);
}

// The reference's second stage over 32 warp sums red[0..31] (warp_sum: xor 16, 8, 4, 2, 1 of the warp index),
// evaluated with lane l holding red[(l & 24) | quad_of_lane(l & 7)]: the warp-index xors are then lane xor 16, 8,
// 7, 2, 1. All 32 lanes of each half-wave return the total.
__device__ __forceinline__ float red32_sum(const float* red) {
  const int l = __lane_id() & 31;
  float v = red[(l & 24) | quad_of_lane(l & 7)];
  v += lane_xor<16>(v);
  v += lane_xor<8>(v);
  v += lane_xor<7>(v);
  v += lane_xor<2>(v);
  v += lane_xor<1>(v);
  return v;
}

}  // namespace q27h
