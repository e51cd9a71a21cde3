/* CPU oracle of the Gated-DeltaNet recurrence (gdn_step): TEST INFRASTRUCTURE ONLY, never linked by the product.
 *
 * Restates the delta rule of the reference's gdn_step_kernel / gdn_prefill_kernel (src/ops.cu:449-572, dispatch
 * src/ops.cu:784-793) in the float-operation order of this library's kernel, which is the contract:
 *   per (head h, value column col), state column S[.][col] split in Q27O_GDN_PARTS parts of E = 128 / parts rows
 *   (part p: rows E p .. E p + E - 1);
 *   per token: part sums kq[i & 3] = fmaf(S[i], k[i], kq[i & 3]) (i ascending inside the part),
 *   P_p = (kq0 + kq1) + (kq2 + kq3); the P_p are added by the xor butterfly with masks 1, 2, 7 (and 8 for 16 parts),
 *   P_p <- P_p + P_{p ^ m};
 *   delta = (v - e^g kv) beta, S[i] = fmaf(k[i], delta, e^g S[i]), the same sums over S[i] q[i] give at,
 *   o = at scale.
 * The fused multiply-adds are part of the contract (as the reference's nvcc build contracts these products).
 * The reference's two kernels use two different orders (32 lanes x 4 and 8 parts x 16), so no single order is the
 * reference's; parity with its mathematics is pinned by tests against a float64 recurrence, and the snapshot /
 * flip plane semantics against the reference's dispatch. e^g is q27o_expf. */
#include <math.h>
#include <stddef.h>

#include "q27_oracle.h"

#ifndef Q27O_GDN_PARTS
#define Q27O_GDN_PARTS 16
#endif

static float parts_sum(const float* P, int parts) {
  float v[16], w[16];
  static const int masks[4] = {1, 2, 7, 8};
  for (int p = 0; p < parts; p++) v[p] = P[p];
  for (int s = 0; s < (parts == 16 ? 4 : 3); s++) {
    for (int p = 0; p < parts; p++) w[p] = v[p] + v[p ^ masks[s]];
    for (int p = 0; p < parts; p++) v[p] = w[p];
  }
  return v[0];  // every part holds the same value: each step adds a pair's two values in either order
}

static float col_dot(const float* s, const float* x, int parts) {
  const int E = 128 / parts;
  float P[16];
  for (int p = 0; p < parts; p++) {
    float kq[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int i = 0; i < E; i++) kq[i & 3] = fmaf(s[E * p + i], x[E * p + i], kq[i & 3]);
    P[p] = (kq[0] + kq[1]) + (kq[2] + kq[3]);
  }
  return parts_sum(P, parts);
}

/* gdn_step (src/ops.h:40-45): planes [4][H][128 col][128 i]; read plane in_plane; o [T][H][128].
 * flip = 0: plane t after token t when snapshots, else plane T - 1 after the last token (T <= 4).
 * flip = 1: the final state to plane (in_plane == 0 ? 1 : 0) only. Returns 0, or -1 on a bad shape. */
int q27o_gdn_step_parts(int parts, const float* q, const float* k, const float* v, int stride, const float* g,
                        const float* beta, float* planes, int in_plane, float* o, int H, int HK, int T, float scale,
                        int snapshots, int flip) {
  if (parts != 8 && parts != 16) return -1;
  if (H <= 0 || HK <= 0 || T < 0 || (!flip && T > 4)) return -1;
  if (T == 0) return 0;
  const size_t plane_sz = (size_t)H * 128 * 128;
  const int out_plane = flip ? (in_plane == 0 ? 1 : 0) : T - 1;
  float s[128];
  for (int h = 0; h < H; h++) {
    const int kh = h % HK;
    for (int col = 0; col < 128; col++) {
      const size_t soff = ((size_t)h * 128 + col) * 128;
      for (int i = 0; i < 128; i++) s[i] = planes[(size_t)in_plane * plane_sz + soff + i];
      for (int t = 0; t < T; t++) {
        const float* qt = q + (size_t)t * stride + kh * 128;
        const float* kt = k + (size_t)t * stride + kh * 128;
        const float gv = q27o_expf(g[(size_t)t * H + h]);
        const float bv = beta[(size_t)t * H + h];
        const float kv = col_dot(s, kt, parts);
        const float delta = (v[(size_t)t * stride + h * 128 + col] - gv * kv) * bv;
        for (int i = 0; i < 128; i++) s[i] = fmaf(kt[i], delta, gv * s[i]);
        o[((size_t)t * H + h) * 128 + col] = col_dot(s, qt, parts) * scale;
        if (!flip && snapshots && t < T - 1)
          for (int i = 0; i < 128; i++) planes[(size_t)t * plane_sz + soff + i] = s[i];
      }
      for (int i = 0; i < 128; i++) planes[(size_t)out_plane * plane_sz + soff + i] = s[i];
    }
  }
  return 0;
}

int q27o_gdn_step(const float* q, const float* k, const float* v, int stride, const float* g, const float* beta,
                  float* planes, int in_plane, float* o, int H, int HK, int T, float scale, int snapshots, int flip) {
  return q27o_gdn_step_parts(Q27O_GDN_PARTS, q, k, v, stride, g, beta, planes, in_plane, o, H, HK, T, scale, snapshots,
                             flip);
}
