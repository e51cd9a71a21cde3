// Attention input stage (attn_prep): per-head RMSNorm of q and k, partial NeoX rotary (plain positions or
// IMRoPE sections), and the K/V cache write as f16 or q8_0.
//
// Lane p of a wave holds 4 head dims in the 32-value block layout of q27h_device.h (16-byte loads and stores). The reference's
// 256-thread block_sum (src/ops.cu:609) is rebuilt from the same operands: per virtual warp of 32 dims
// (8 lanes) vwarp_sum4, then the second stage over the 8 warp sums w_g (lanes 8g..8g+7), whose reference tree
// ((w0+w4)+(w2+w6)) + ((w1+w5)+(w3+w7)) is lane xor 32, xor 16, xor 8. The rotary partner of dim j < 32 is dim
// j + 32, i.e. the same lane of the next 8-lane group, lane p ^ 8 (a DPP row rotate). Angles are (float)p * freq[j] with freq[j] = theta_scale^j taken
// once on the host; sin and cos come from the shared double-precision routine.
#include <cmath>

#include "q27h_device.h"
#include "q27h_internal.h"

namespace q27h {
namespace {
#ifndef Q27H_NT_ATTN
#define Q27H_NT_ATTN 1
#endif
constexpr bool kAttnNT = Q27H_NT_ATTN;  // nontemporal qn stores (measured in the prefill pass)

struct RopeFreqs {
  float f[32];
};


// One wave per (token, group of HPW heads). Batches: HPW = 4, one workgroup of 7 waves per token (TOKWG below), wave w
// taking heads w, w + 7, w + 14, w + 21, so the 4 K heads with their q8/f16 cache work sit in 4 different waves
// (2048 tokens: 23.9 us against 26.3 us for 2 heads per wave, both one workgroup per token, and 26.2 us for 2 heads per
// wave with every wave evaluating the angles). A few tokens: HPW = 1 and four independent waves per workgroup,
// where the shorter chain per wave matters more than loads in flight; every wave then evaluates the 32 angles of
// its token (lane j < 32 takes pair j) and hands them to the lanes that need them with ds_bpermute. The head vectors
// of the whole group are loaded before any arithmetic.
#ifndef Q27H_ATTN_HPW
#define Q27H_ATTN_HPW 4
#endif

// TOKWG: one workgroup per token (its waves = the token's head groups). Wave 0 evaluates the 32 angles once for the
// token and hands them out through LDS, instead of every wave of the token evaluating them: the rotary setup (the
// frequency select and the double-precision sin / cos) was about a third of each wave's VALU instructions.
template <int HPW, bool TOKWG>
__global__ void __launch_bounds__(1024) attn_prep_kernel(const float* __restrict__ qg, const float* __restrict__ k,
                                                        const float* __restrict__ v, const float* __restrict__ q_norm,
                                                        const float* __restrict__ k_norm, float* __restrict__ qn,
                                                        void* __restrict__ kcache, void* __restrict__ vcache,
                                                        const int* __restrict__ dpos0, int T, float eps, RopeFreqs fr,
                                                        int nqh, int nkvh, int n_ctx, int q8, const int* __restrict__ rope3,
                                                        const int* __restrict__ rdelta) {
  const int nh = nqh + nkvh;
  const int wpt = (nh + HPW - 1) / HPW;  // waves per token
  int tok, hw;  // heads hw, hw + wpt, hw + 2 wpt, ...: the K heads (the last ones) fall in different waves
  if constexpr (TOKWG) {
    tok = blockIdx.x;  // blockDim.x = 64 wpt: every wave of the workgroup has a head group
    hw = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  } else {
    const int wave = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar registers
    if (wave >= T * wpt) return;  // whole waves leave together
    tok = wave / wpt;
    hw = wave % wpt;
  }
  const int nhw = (nh - hw + wpt - 1) / wpt;
  const int p = threadIdx.x & 63;
  const int off = 32 * (p >> 3) + block_offset(p);  // this lane's 4 head dims (32-value block layout)
  const int pos = *dpos0 + tok;  // cache row
  // ---- loads of the whole group first, branch-free (a missing head of the last group re-reads head hw)
  float4 xin[HPW], vin[HPW];
#pragma unroll
  for (int i = 0; i < HPW; i++) {
    const int hb = i < nhw ? hw + i * wpt : hw;
    const float* src = hb < nqh ? qg + ((size_t)tok * nqh + hb) * 512 : k + ((size_t)tok * nkvh + (hb - nqh)) * 256;
    xin[i] = ld4_nt(src + off);
  }
#pragma unroll
  for (int i = 0; i < HPW; i++) {
    const int hb = hw + i * wpt;
    if (i < nhw && hb >= nqh) vin[i] = ld4_nt(v + ((size_t)tok * nkvh + (hb - nqh)) * 256 + off);
  }
  const float4 qw = ld4(q_norm + off);
  const float4 kw = ld4((nkvh ? k_norm : q_norm) + off);
  // ---- rotary angles of the token, lane j < 32 evaluating pair j, from scalar loads and kernel arguments only
  // (no wait on the vector loads above, so the sin/cos run while the head vectors are in flight)
  const int j32 = p & 31;
  auto angle = [&](float& sn_j, float& cs_j) {
    int rp;
    if (rope3) {
      const int r0 = rope3[tok * 3], r1 = rope3[tok * 3 + 1], r2 = rope3[tok * 3 + 2];
      const int m = j32 % 3;
      rp = m == 0 ? r0 : m == 1 ? r1 : r2;
    } else {
      rp = pos - (rdelta ? *rdelta : 0);
    }
    float fj = fr.f[0];  // fr.f[j32], selected from the argument registers
#pragma unroll
    for (int m = 1; m < 32; m++) {
      float fm = fr.f[m];
      asm("" : "+s"(fm));  // keeps the selects (no indexed load from the argument segment, which would wait behind the head loads)
      fj = j32 == m ? fm : fj;
    }
    q27_sincos((float)rp * fj, &sn_j, &cs_j);
  };
  float snc[4], csc[4];
  if constexpr (TOKWG) {
    __shared__ float s_sc[2][32];
    if (hw == 0 && p < 32) {
      float sn_j, cs_j;
      angle(sn_j, cs_j);
      s_sc[0][p] = sn_j;
      s_sc[1][p] = cs_j;
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < 4; c++) {
      snc[c] = s_sc[0][(off + c) & 31];
      csc[c] = s_sc[1][(off + c) & 31];
    }
  } else {
    float sn_j, cs_j;
    angle(sn_j, cs_j);
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const int j = (off + c) & 31;
      snc[c] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(j << 2, __builtin_bit_cast(int, sn_j)));
      csc[c] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(j << 2, __builtin_bit_cast(int, cs_j)));
    }
  }
  const bool valid = pos >= 0 && pos < n_ctx;  // uniform over the wave
  const size_t so = (size_t)nkvh * n_ctx * 256;
  // RMSNorm over the 256 dims, for every head of the group first (independent reductions whose lane exchanges
  // overlap): 8 virtual warps of 32 (8 lanes each), then ((w0+w4)+(w2+w6)) + ((w1+w5)+(w3+w7))
  float scale[HPW];
#pragma unroll
  for (int i = 0; i < HPW; i++) {
    float sq[4] = {xin[i].x * xin[i].x, xin[i].y * xin[i].y, xin[i].z * xin[i].z, xin[i].w * xin[i].w};
    float t = vwarp_sum4(sq);
    t = t + lane_xor32(t);
    t += lane_xor<16>(t);
    t += lane_xor<8>(t);
    scale[i] = 1.0f / __builtin_sqrtf(t / 256.0f + eps);
  }
#pragma unroll
  for (int i = 0; i < HPW; i++) {
    if (i >= nhw) break;
    const int hb = hw + i * wpt;
    const bool isq = hb < nqh;
    const float x[4] = {xin[i].x, xin[i].y, xin[i].z, xin[i].w};
    const float sc = scale[i];
    const float4 wv = isq ? qw : kw;
    const float ww[4] = {wv.x, wv.y, wv.z, wv.w};
    float buf[4], out[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
      buf[c] = sc * x[c] * ww[c];
      out[c] = buf[c];
    }
    // NeoX rotation of (j, j + 32), j < 32: the partner of lane p < 16 is lane p ^ 8
    float partner[4];
#pragma unroll
    for (int c = 0; c < 4; c++) partner[c] = lane_xor<8>(buf[c]);
    // lanes 0..7: x0 * c - x1 * s; lanes 8..15: x0 * s + x1 * c (selects, no divergent branch)
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const float bc = buf[c] * csc[c], ps = partner[c] * snc[c];
      const float r0 = bc - ps, r1 = ps + bc;
      out[c] = p < 8 ? r0 : p < 16 ? r1 : buf[c];
    }
    if (isq) {
      st4<kAttnNT>(qn + ((size_t)tok * nqh + hb) * 256 + off, out[0], out[1], out[2], out[3]);
      continue;
    }
    const int kh = hb - nqh;
    const float vv[4] = {vin[i].x, vin[i].y, vin[i].z, vin[i].w};
    const size_t row = (size_t)kh * n_ctx + (size_t)(valid ? pos : 0);
    if (!q8) {
      if (!valid) continue;
      uint16_t* kc = (uint16_t*)kcache + row * 256 + off;
      uint16_t* vc = (uint16_t*)vcache + row * 256 + off;
      *(uint2*)kc = make_uint2((uint32_t)f2h_bits(out[0]) | ((uint32_t)f2h_bits(out[1]) << 16),
                               (uint32_t)f2h_bits(out[2]) | ((uint32_t)f2h_bits(out[3]) << 16));
      *(uint2*)vc = make_uint2((uint32_t)f2h_bits(vv[0]) | ((uint32_t)f2h_bits(vv[1]) << 16),
                               (uint32_t)f2h_bits(vv[2]) | ((uint32_t)f2h_bits(vv[3]) << 16));
      continue;
    }
    // q8_0 per 32 dims (8 lanes): d = amax / 127, q = roundf(x * (d ? 1/d : 0)) (src/ops.cu:636-646)
    float ak = __builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(out[0]), __builtin_fabsf(out[1])),
                               __builtin_fmaxf(__builtin_fabsf(out[2]), __builtin_fabsf(out[3])));
    float av = __builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(vv[0]), __builtin_fabsf(vv[1])),
                               __builtin_fmaxf(__builtin_fabsf(vv[2]), __builtin_fabsf(vv[3])));
    ak = __builtin_fmaxf(ak, lane_xor<7>(ak));
    av = __builtin_fmaxf(av, lane_xor<7>(av));
    ak = __builtin_fmaxf(ak, lane_xor<2>(ak));
    av = __builtin_fmaxf(av, lane_xor<2>(av));
    ak = __builtin_fmaxf(ak, lane_xor<1>(ak));
    av = __builtin_fmaxf(av, lane_xor<1>(av));
    if (!valid) continue;
    const float dk = ak / 127.f, dv = av / 127.f;
    const float ik = dk != 0.0f ? 1.0f / dk : 0.0f, iv = dv != 0.0f ? 1.0f / dv : 0.0f;
    int8_t* kq = (int8_t*)kcache + row * 256 + off;
    int8_t* vq = (int8_t*)vcache + row * 256 + off;
    *(uint32_t*)kq = pack4_i8((int)__builtin_roundf(out[0] * ik), (int)__builtin_roundf(out[1] * ik),
                              (int)__builtin_roundf(out[2] * ik), (int)__builtin_roundf(out[3] * ik));
    *(uint32_t*)vq = pack4_i8((int)__builtin_roundf(vv[0] * iv), (int)__builtin_roundf(vv[1] * iv),
                              (int)__builtin_roundf(vv[2] * iv), (int)__builtin_roundf(vv[3] * iv));
    if ((p & 7) == 0) {
      ((uint16_t*)((uint8_t*)kcache + so))[row * 8 + (p >> 3)] = f2h_bits(dk);
      ((uint16_t*)((uint8_t*)vcache + so))[row * 8 + (p >> 3)] = f2h_bits(dv);
    }
  }
}

}  // namespace
}  // namespace q27h

using namespace q27h;

extern "C" size_t q27h_kv_cache_bytes(int nkvh, int n_ctx, int q8) {
  return q8 ? (size_t)nkvh * (size_t)n_ctx * (256 + 16) : (size_t)nkvh * (size_t)n_ctx * 256 * 2;
}

extern "C" int q27h_attn_prep(const float* qg, const float* k, const float* v, const float* q_norm, const float* k_norm,
                              float* qn, void* kcache, void* vcache, const int* pos0, int T, float eps, float theta_scale,
                              int nqh, int nkvh, int n_ctx, int q8, q27h_stream_t s, const void* pf, size_t pf_bytes,
                              const int* rope3, const int* rdelta) {
  (void)pf;
  (void)pf_bytes;
  if (T < 0 || nqh < 0 || nkvh < 0 || n_ctx <= 0) return fail(Q27H_ERR_SHAPE, "attn_prep: bad shape");
  if (T == 0 || nqh + nkvh == 0) return Q27H_OK;
  if (!qg || !q_norm || !qn || !pos0 || (nkvh && (!k || !v || !k_norm || !kcache || !vcache)))
    return fail(Q27H_ERR_ARG, "attn_prep: null pointer");
  if (!aligned16(qg) || !aligned16(q_norm) || !aligned16(qn) || (nkvh && (!aligned16(k) || !aligned16(v) ||
      !aligned16(k_norm) || !aligned16(kcache) || !aligned16(vcache))))
    return fail(Q27H_ERR_ARG, "attn_prep: tensors need 16-byte alignment");
  RopeFreqs fr;
  for (int j = 0; j < 32; j++) fr.f[j] = powf(theta_scale, (float)j);
  const int nh = nqh + nkvh;
  if ((long)T * nh < 2048) {
    const long waves = (long)T * nh;
    hipLaunchKernelGGL((attn_prep_kernel<1, false>), dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, stream_of(s), qg, k,
                       v, q_norm, k_norm, qn, kcache, vcache, pos0, T, eps, fr, nqh, nkvh, n_ctx, q8, rope3, rdelta);
  } else {
    constexpr int hpw = Q27H_ATTN_HPW;
    const int wpt = (nh + hpw - 1) / hpw;
    if (wpt <= 16)
      hipLaunchKernelGGL((attn_prep_kernel<hpw, true>), dim3((unsigned)T), dim3(64 * wpt), 0, stream_of(s), qg, k, v, q_norm,
                         k_norm, qn, kcache, vcache, pos0, T, eps, fr, nqh, nkvh, n_ctx, q8, rope3, rdelta);
    else
      hipLaunchKernelGGL((attn_prep_kernel<hpw, false>), dim3((unsigned)(((long)T * wpt + 3) / 4)), dim3(256), 0, stream_of(s),
                         qg, k, v, q_norm, k_norm, qn, kcache, vcache, pos0, T, eps, fr, nqh, nkvh, n_ctx, q8, rope3, rdelta);
  }
  return check_launch("attn_prep");
}
