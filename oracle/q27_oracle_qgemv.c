/* CPU oracle of the decode GEMV over quantized weights: TEST INFRASTRUCTURE ONLY.
 *
 * y[c][n] = sum_k W[n][k] x[c][k] for ncols <= 4 activation columns given as q8_1 (xq int8 [c][K], xd [c][K/32]),
 * W as raw GGUF blocks (N rows of K/256 blocks). It restates the reference's decode GEMV (src/qgemv.cu:369-560
 * dot_chunk, src/qmat.h:44-46): per row, per 256-weight block b and 32-weight sub-block s an exact integer dot of the
 * block's quants with the 32 int8 activations (llama.cpp vecdotq semantics), turned into a float contribution
 * t(b, s) with the reference's float expression of that type. Only the summation order of the t is this build's own
 * (the reference's depends on the SM count through its split-K choice, src/qgemv.cu:743-753):
 *   - W "waves" per 8-row tile (q27o_qgemv_waves of the type, K and the launch's column count), 64 lanes each, lane = 8 lb + s; slot g = 8 w + lb takes the
 *     blocks g, g + 8 W, g + 16 W, ... in ascending order: acc = 0, acc = acc + t(b, s);
 *   - the 64 lane sums of a wave are added as an xor butterfly (lane xor 32, 16, 8, 4, 2, 1);
 *   - the wave sums are added in wave order: ((P0 + P1) + P2) + ...
 * The GPU kernel (qwen27-engine_amd/csrc/qgemv.hip) adds the same operands in the same order.
 * Block formats: ggml block_q2_K / q4_K / q6_K / iq2_xxs / iq2_xs / iq2_s / iq3_xxs / iq3_s / iq4_xs / iq1_m
 * (ggml-common.h), the dequantization order of src/requant.cpp:68-114 (Q6_K, Q4_K) and ggml's dequantize_row_*; the
 * integer scale rules of the IQ2 / IQ3_XXS types, including their truncating divisions, are the reference's
 * (src/qgemv.cu:395-420, 492-545).
 * Parity: pinned by tests/test_oracle_qgemv.py (exact-integer cases against numpy dequantizers, a float64
 * dequantize-and-dot bound, the waves rule shared with the library). */
#include <stdint.h>
#include <string.h>

#include "q27_oracle.h"

static const uint32_t kIQ3SGrid[512] = {
#include "../qwen27-engine_amd/csrc/iq3s_grid.inc"
};
static const int8_t kIQ4NL[16] = {
#include "../qwen27-engine_amd/csrc/iq4nl_values.inc"
};
static const uint64_t kIQ2XXSGrid[256] = {
#include "../qwen27-engine_amd/csrc/iq2xxs_grid.inc"
};
static const uint64_t kIQ2XSGrid[512] = {
#include "../qwen27-engine_amd/csrc/iq2xs_grid.inc"
};
static const uint64_t kIQ2SGrid[1024] = {
#include "../qwen27-engine_amd/csrc/iq2s_grid.inc"
};
static const uint32_t kIQ3XXSGrid[256] = {
#include "../qwen27-engine_amd/csrc/iq3xxs_grid.inc"
};
static const uint32_t kIQ1SGrid[2048] = {
#include "../qwen27-engine_amd/csrc/iq1s_grid.inc"
};

enum {
  T_Q2_K = 10, T_Q4_K = 12, T_Q6_K = 14, T_IQ2_XXS = 16, T_IQ2_XS = 17, T_IQ3_XXS = 18, T_IQ3_S = 21, T_IQ2_S = 22,
  T_IQ4_XS = 23, T_IQ1_M = 29
};

/* 7 sign bits plus the parity bit that makes the count of negative signs even (ggml ksigns_iq2xs) */
static int ksigns(int v7) { return v7 | ((__builtin_popcount(v7) & 1) << 7); }
/* sum over the 8 magnitudes of a 64-bit grid entry (one byte each) times the signed activations */
static int dot8(uint64_t g, int signs, const int8_t* u) {
  int s = 0;
  for (int j = 0; j < 8; j++) {
    const int mag = (int)((g >> (8 * j)) & 0xFF);
    s += ((signs >> j) & 1 ? -mag : mag) * u[j];
  }
  return s;
}

int q27o_qgemv_block_bytes(int type) {
  switch (type) {
    case T_Q4_K: return 144;
    case T_Q6_K: return 210;
    case T_IQ3_S: return 110;
    case T_IQ4_XS: return 136;
    case T_Q2_K: return 84;
    case T_IQ2_XXS: return 66;
    case T_IQ2_XS: return 74;
    case T_IQ3_XXS: return 98;
    case T_IQ2_S: return 82;
    case T_IQ1_M: return 56;
    default: return 0;
  }
}

/* Waves per 8-row tile: a function of the type, K and the column count only, so results do not depend on the device.
 * One column, and two for all types but IQ3_XXS / IQ3_S / IQ1_M: ceil(K / 2048) up to K = 32768 (at most 16);
 * otherwise at most 4; K > 32768: 4. */
int q27o_qgemv_waves(int type, int K, int ncols) {
  const int w = (K / 256 + 7) / 8;
  const int wide = ncols == 1 || (ncols == 2 && type != 18 && type != 21 && type != 29);
  const int cap = wide ? 16 : 4;
  return w < 1 ? 1 : w > 16 ? 4 : w > cap ? cap : w;
}

static float h2f(const uint8_t* p) { return q27o_h2f((uint16_t)(p[0] | (p[1] << 8))); }

/* Contribution of sub-block s (32 weights) of one raw block to column activations u[32] with scale dy. */
static float chunk_t(int type, const uint8_t* blk, int s, const int8_t* u, float dy) {
  if (type == T_Q4_K) {
    /* d, dmin, scales[12], qs[128]; weights of sub s: nibble (s & 1) of qs[32 (s / 2) + l] */
    const float d = h2f(blk), dmin = h2f(blk + 2);
    const uint8_t* sc = blk + 4;
    const uint8_t* qs = blk + 16 + 32 * (s / 2);
    int scv, mv;
    if (s < 4) {
      scv = sc[s] & 63;
      mv = sc[s + 4] & 63;
    } else {
      scv = (sc[s + 4] & 0xF) | ((sc[s - 4] >> 6) << 4);
      mv = (sc[s + 4] >> 4) | ((sc[s] >> 6) << 4);
    }
    int sumi = 0, s8 = 0;
    for (int l = 0; l < 32; l++) {
      sumi += ((qs[l] >> (4 * (s & 1))) & 0xF) * u[l];
      s8 += u[l];
    }
    return d * (dy * (float)(sumi * scv)) - dmin * (dy * (float)(s8 * mv));
  }
  if (type == T_Q6_K) {
    /* ql[128], qh[64], scales[16] (int8), d; sub s = 4 n + j covers weights 128 n + 32 j + l */
    const int n = s / 4, j = s % 4;
    const uint8_t* ql = blk + 64 * n + 32 * (j & 1);
    const uint8_t* qh = blk + 128 + 32 * n;
    const int8_t* scales = (const int8_t*)(blk + 192 + 8 * n + 2 * j);
    const float d = h2f(blk + 208);
    int sa = 0, sb = 0, s8a = 0, s8b = 0;
    for (int l = 0; l < 32; l++) {
      const int lo = j < 2 ? (ql[l] & 0xF) : (ql[l] >> 4);
      const int q = lo | (((qh[l] >> (2 * j)) & 3) << 4);
      if (l < 16) { sa += q * u[l]; s8a += u[l]; }
      else { sb += q * u[l]; s8b += u[l]; }
    }
    const int si = (sa - 32 * s8a) * scales[0] + (sb - 32 * s8b) * scales[1];
    return d * (dy * (float)si);
  }
  if (type == T_IQ4_XS) {
    /* d, scales_h (u16), scales_l[4], qs[128]; sub s: level = kvalues[nibble], low nibbles weights 0..15 */
    const float d = h2f(blk);
    const int sh = blk[2] | (blk[3] << 8);
    const int ls = (((blk[4 + s / 2] >> (4 * (s & 1))) & 0xF) | (((sh >> (2 * s)) & 3) << 4)) - 32;
    const uint8_t* qs = blk + 8 + 16 * s;
    int sumi = 0;
    for (int l = 0; l < 16; l++) {
      sumi += kIQ4NL[qs[l] & 0xF] * u[l];
      sumi += kIQ4NL[qs[l] >> 4] * u[l + 16];
    }
    return (d * dy) * (float)(sumi * ls);
  }
  if (type == T_IQ3_S) {
    /* d, qs[64], qh[8], signs[32], scales[4]; sub s: grid k = 0..7 covers weights 4 k .. 4 k + 3 */
    const float d = h2f(blk);
    const uint8_t* qs = blk + 2 + 8 * s;
    const int qh = blk[66 + s];
    const uint8_t* signs = blk + 74 + 4 * s;
    const int mul = 1 + 2 * ((blk[106 + s / 2] >> (4 * (s & 1))) & 0xF);
    int sumi = 0;
    for (int k = 0; k < 8; k++) {
      const int idx = qs[k] | ((qh << (8 - k)) & 256);
      const uint32_t g = kIQ3SGrid[idx];
      for (int jj = 0; jj < 4; jj++) {
        const int mag = (int)((g >> (8 * jj)) & 0xFF);
        const int neg = (signs[k / 2] >> (jj + 4 * (k & 1))) & 1;
        sumi += (neg ? -mag : mag) * u[4 * k + jj];
      }
    }
    return (d * dy) * (float)(sumi * mul);
  }
  if (type == T_Q2_K) {
    /* scales[16], qs[64], d, dmin; sub s = 4 n + j: weights 128 n + 32 j + l = (qs[32 n + l] >> 2 j) & 3, the two
     * 16-weight halves with scale byte scales[8 n + 2 j + h] (low nibble scale, high nibble min) */
    const int n = s / 4, j = s % 4;
    const float d = h2f(blk + 80), dmin = h2f(blk + 82);
    const uint8_t g0 = blk[8 * n + 2 * j], g1 = blk[8 * n + 2 * j + 1];
    int sa = 0, sb = 0, s8a = 0, s8b = 0;
    for (int l = 0; l < 32; l++) {
      const int q = (blk[16 + 32 * n + l] >> (2 * j)) & 3;
      if (l < 16) { sa += q * u[l]; s8a += u[l]; }
      else { sb += q * u[l]; s8b += u[l]; }
    }
    const int sd = sa * (g0 & 0xF) + sb * (g1 & 0xF);
    const int smn = s8a * (g0 >> 4) + s8b * (g1 >> 4);
    return d * (dy * (float)sd) - dmin * (dy * (float)smn);
  }
  if (type == T_IQ2_XXS) {
    /* d, then per sub-block 4 grid index bytes and a word of 4 x 7 sign bits + a 4-bit scale (top bits) */
    const float d = h2f(blk);
    const uint8_t* q = blk + 2 + 8 * s;
    const uint32_t aux = (uint32_t)q[4] | ((uint32_t)q[5] << 8) | ((uint32_t)q[6] << 16) | ((uint32_t)q[7] << 24);
    int sumi = 0;
    for (int p = 0; p < 4; p++) sumi += dot8(kIQ2XXSGrid[q[p]], ksigns((aux >> (7 * p)) & 0x7F), u + 8 * p);
    const int ls = (int)((aux >> 27) | 1);
    return (d * dy) * (float)(sumi * ls / 8);
  }
  if (type == T_IQ2_XS || type == T_IQ2_S) {
    const float d = h2f(blk);
    int s0 = 0, s1 = 0, lsb;
    for (int p = 0; p < 4; p++) {
      int gi, sb;
      if (type == T_IQ2_XS) {  /* d, qs[32] (u16: 9-bit grid index, 7 sign bits), scales[8] */
        const int q16 = blk[2 + 8 * s + 2 * p] | (blk[3 + 8 * s + 2 * p] << 8);
        gi = q16 & 0x1FF;
        sb = ksigns(q16 >> 9);
      } else {  /* d, qs[32], signs[32], qh[8], scales[8]: 10-bit index = qs | 2 bits of qh */
        gi = blk[2 + 4 * s + p] | ((blk[66 + s] << (8 - 2 * p)) & 0x300);
        sb = blk[34 + 4 * s + p];
      }
      const int v = dot8(type == T_IQ2_XS ? kIQ2XSGrid[gi] : kIQ2SGrid[gi], sb, u + 8 * p);
      if (p < 2) s0 += v;
      else s1 += v;
    }
    lsb = blk[(type == T_IQ2_XS ? 66 : 74) + s];
    const int si = (s0 * (lsb & 0xF) + s1 * (lsb >> 4) + (s0 + s1) / 2) / 4;
    return (d * dy) * (float)si;
  }
  if (type == T_IQ3_XXS) {
    /* d, qs[64] (grid indices, 8 per sub-block), then per sub-block a word of 4 x 7 sign bits + 4-bit scale */
    const float d = h2f(blk);
    const uint8_t* qs = blk + 2 + 8 * s;
    const uint8_t* a = blk + 66 + 4 * s;
    const uint32_t aux = (uint32_t)a[0] | ((uint32_t)a[1] << 8) | ((uint32_t)a[2] << 16) | ((uint32_t)a[3] << 24);
    int sumi = 0;
    for (int p = 0; p < 4; p++) {
      const int sb = ksigns((aux >> (7 * p)) & 0x7F);
      const uint64_t g = (uint64_t)kIQ3XXSGrid[qs[2 * p]] | ((uint64_t)kIQ3XXSGrid[qs[2 * p + 1]] << 32);
      sumi += dot8(g, sb, u + 8 * p);
    }
    const int ls = (int)(aux >> 28);
    const int si = (ls * sumi + sumi / 2) / 2;
    return (d * dy) * (float)si;
  }
  if (type == T_IQ1_M) {
    /* qs[32], qh[16], scales[8] (4 x u16; the fp16 super-block scale is their four top nibbles). Grid entries hold
     * 8 nibbles g (value + 1); each group of 8 weights adds delta * (sum of its activations) with delta = -7/8 or
     * -9/8 by bit 3 of the group's qh nibble. */
    uint16_t s16[4];
    for (int k = 0; k < 4; k++) s16[k] = (uint16_t)(blk[48 + 2 * k] | (blk[49 + 2 * k] << 8));
    const uint16_t dh = (uint16_t)((s16[0] >> 12) | ((s16[1] >> 8) & 0x00F0) | ((s16[2] >> 4) & 0x0F00) | (s16[3] & 0xF000));
    const float dw = q27o_h2f(dh);
    const int qh16 = blk[32 + 2 * s] | (blk[33 + 2 * s] << 8);
    const int sc6 = (s16[s / 2] >> (6 * (s % 2))) & 63;
    int si[2] = {0, 0};
    float sf[2] = {0.0f, 0.0f};
    for (int p = 0; p < 4; p++) {
      const int qhl = (qh16 >> (4 * p)) & 0xF;
      const uint32_t grid = kIQ1SGrid[blk[4 * s + p] | ((qhl & 7) << 8)];
      int sy = 0, dotp = 0;
      for (int jj = 0; jj < 8; jj++) {
        /* nibble order of the GPU grid: bytes of (grid & 0x0F0F0F0F) are weights 0..3, of (grid >> 4) weights 4..7 */
        const int g = jj < 4 ? (int)((grid >> (8 * jj)) & 0xF) : (int)((grid >> (8 * (jj - 4) + 4)) & 0xF);
        dotp += g * u[8 * p + jj];
        sy += u[8 * p + jj];
      }
      const float delta = -1.0f + 0.125f - (float)(qhl & 0x08) * (2.0f * 0.125f / 8.0f);
      si[p / 2] += dotp;
      sf[p / 2] += delta * (float)sy;
    }
    const int sc0 = 2 * (sc6 & 7) + 1, sc1 = 2 * ((sc6 >> 3) & 7) + 1;
    return (dw * dy) * ((((float)si[0] + sf[0]) * (float)sc0) + (((float)si[1] + sf[1]) * (float)sc1));
  }
  return 0.0f;
}

int q27o_qgemv(int type, const uint8_t* raw, int N, int K, const int8_t* xq, const float* xd, float* y, int ncols) {
  const int bb = q27o_qgemv_block_bytes(type);
  if (!bb || N % 8 || K % 256 || ncols < 1 || ncols > 4) return -1;
  const int nb = K / 256;
  for (int n = 0; n < N; n++) {
    const uint8_t* row = raw + (size_t)n * nb * bb;
    for (int c = 0; c < ncols; c++) {
      /* three columns run as a launch of two columns and one of one */
      const int W = q27o_qgemv_waves(type, K, ncols == 3 ? (c < 2 ? 2 : 1) : ncols);
      const int8_t* xr = xq + (size_t)c * K;
      const float* dr = xd + (size_t)c * (K / 32);
      float total = 0.0f;
      for (int w = 0; w < W; w++) {
        float v[64];
        for (int lane = 0; lane < 64; lane++) {
          const int lb = lane >> 3, s = lane & 7;
          float acc = 0.0f;
          for (int b = 8 * w + lb; b < nb; b += 8 * W) acc = acc + chunk_t(type, row + (size_t)b * bb, s, xr + b * 256 + 32 * s, dr[b * 8 + s]);
          v[lane] = acc;
        }
        for (int o = 32; o >= 1; o >>= 1) {
          float t[64];
          for (int l = 0; l < 64; l++) t[l] = v[l] + v[l ^ o];
          memcpy(v, t, sizeof v);
        }
        total = w == 0 ? v[0] : total + v[0];
      }
      y[(size_t)c * N + n] = total;
    }
  }
  return 0;
}
