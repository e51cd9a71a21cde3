/* CPU oracle of the decode GEMV over quantized weights: TEST INFRASTRUCTURE ONLY.
 *
 * y[c][n] = sum_k W[n][k] x[c][k] for ncols <= 4 activation columns given as q8_1 (xq int8 [c][K], xd [c][K/32]),
 * W as raw GGUF blocks (N rows of K/256 blocks). It restates the reference's decode GEMV (src/qgemv.cu:369-560
 * dot_chunk, src/qmat.h:44-46): per row, per 256-weight block b and 32-weight sub-block s an exact integer dot of the
 * block's quants with the 32 int8 activations (llama.cpp vecdotq semantics), turned into a float contribution
 * t(b, s) with the reference's float expression of that type. Only the summation order of the t is this build's own
 * (the reference's depends on the SM count through its split-K choice, src/qgemv.cu:743-753):
 *   - W "waves" per 8-row tile (q27o_qgemv_waves), 64 lanes each, lane = 8 lb + s; slot g = 8 w + lb takes the
 *     blocks g, g + 8 W, g + 16 W, ... in ascending order: acc = 0, acc = acc + t(b, s);
 *   - the 64 lane sums of a wave are added as an xor butterfly (lane xor 32, 16, 8, 4, 2, 1);
 *   - the wave sums are added in wave order: ((P0 + P1) + P2) + P3.
 * The GPU kernel (qwen27-engine_amd/csrc/qgemv.hip) adds the same operands in the same order.
 * Block formats: ggml block_q4_K / block_q6_K / block_iq4_xs / block_iq3_s (ggml-common.h), the dequantization
 * order of src/requant.cpp:68-114 (Q6_K, Q4_K) and ggml's dequantize_row_iq4_xs / dequantize_row_iq3_s.
 * Parity: pinned by tests/test_oracle_qgemv.py (float64 dequantize-and-dot bound, one-hot integer cases, the
 * summation order replayed in numpy). */
#include <stdint.h>
#include <string.h>

#include "q27_oracle.h"

static const uint32_t kIQ3SGrid[512] = {
#include "../qwen27-engine_amd/csrc/iq3s_grid.inc"
};
static const int8_t kIQ4NL[16] = {
#include "../qwen27-engine_amd/csrc/iq4nl_values.inc"
};

enum { T_Q4_K = 12, T_Q6_K = 14, T_IQ3_S = 21, T_IQ4_XS = 23 };

int q27o_qgemv_block_bytes(int type) {
  switch (type) {
    case T_Q4_K: return 144;
    case T_Q6_K: return 210;
    case T_IQ3_S: return 110;
    case T_IQ4_XS: return 136;
    default: return 0;
  }
}

/* Waves per 8-row tile: a function of the shape only (ceil(K / 2048), at most 4), so results do not depend on the
 * device. */
int q27o_qgemv_waves(int N, int K) {
  (void)N;
  const int w = (K / 256 + 7) / 8;
  return w < 1 ? 1 : w > 4 ? 4 : w;
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
  return 0.0f;
}

int q27o_qgemv(int type, const uint8_t* raw, int N, int K, const int8_t* xq, const float* xd, float* y, int ncols) {
  const int bb = q27o_qgemv_block_bytes(type);
  if (!bb || N % 8 || K % 256 || ncols < 1 || ncols > 4) return -1;
  const int nb = K / 256, W = q27o_qgemv_waves(N, K);
  for (int n = 0; n < N; n++) {
    const uint8_t* row = raw + (size_t)n * nb * bb;
    for (int c = 0; c < ncols; c++) {
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
