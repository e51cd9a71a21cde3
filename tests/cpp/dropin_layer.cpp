// Test helper: call sequences of the reference engine's src/model.cu written against the C++ drop-in headers (a GDN
// layer in decode, :699-742, and prefill, :1210-1225; the fused ops of an attention + FFN prefill layer; a decode
// GEMV whose weights come from a GGUF file), built into a shared library that tests/test_gpu_cpp_dropin.py drives
// through ctypes. It checks that the headers, their default arguments and their exceptions work at run time, not
// only that they compile.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <stdexcept>

#include "q27/ops.h"
#include "q27/prefill.h"
#include "q27/qmat.h"

namespace {
constexpr int E = 5120, D = 128, KH = 16, H = 48, C = 2 * KH * D + H * D;
constexpr float EPS = 1e-6f;

int report(const std::exception& e, char* err, int errlen) {
  std::snprintf(err, (size_t)errlen, "%s", e.what());
  return 1;
}
}  // namespace

// Decode, T <= 4 tokens: x += partial, norm -> h and q8_1; the bf16 alpha / beta projections of h; conv + l2 + gates
// with snapshots; the delta rule with snapshots; gated norm -> q8_1 of o.
extern "C" int dropin_gdn_decode(int T, float* x, const float* partial, const float* w_norm, float* h, int8_t* xq,
                                 float* xd, const __hip_bfloat16* w_alpha, const __hip_bfloat16* w_beta, float* ab,
                                 const float* conv_in, const float* conv_w, float* conv_planes,
                                 const int* plane, float* conv_y, const float* ssm_a,
                                 const float* dt_bias, float* g, float* beta, float* ssm_planes, float* o,
                                 const float* gnorm_w, const float* z, int8_t* oxq, float* oxd, hipStream_t s, char* err,
                                 int errlen) {
  try {
    q27::sum_norm_q8(x, partial, E, T, nullptr, w_norm, EPS, h, xq, xd, s);
    q27::gemv_bf16_pair(w_alpha, w_beta, h, ab, ab + T * H, H, E, T, s);  // src/model.cu:776
    q27::gdn_conv_l2(conv_in, conv_w, conv_planes, plane, conv_y, C, T, true, 2 * KH, EPS, ab, ab + T * H, ssm_a, dt_bias, g,
                     beta, H, s);
    q27::gdn_step(conv_y, conv_y + KH * D, conv_y + 2 * KH * D, C, g, beta, ssm_planes, plane, o, H, KH, T,
                  1.0f / std::sqrt((float)D), true, s);
    q27::gated_rmsnorm_q8(o, gnorm_w, z, oxq, oxd, H * T, EPS, s);
    return 0;
  } catch (const std::exception& e) {
    return report(e, err, errlen);
  }
}

// Prefill of M tokens: conv (flip) + l2 + gates, the delta rule in flip mode, gated norm, then the plane flip.
extern "C" int dropin_gdn_prefill(int M, const float* conv_in, const float* conv_w, float* conv_planes, int* plane,
                                  float* conv_y, const float* a, const float* b, const float* ssm_a, const float* dt_bias,
                                  float* g, float* beta, float* ssm_planes, float* o, const float* gnorm_w, const float* z,
                                  int8_t* oxq, float* oxd, float* oxs, hipStream_t s, char* err, int errlen) {
  try {
    q27::gdn_conv_prefill(conv_in, conv_w, conv_planes, plane, conv_y, C, M, 2 * KH, EPS, a, b, ssm_a, dt_bias, g, beta,
                          H, s);
    q27::gdn_step(conv_y, conv_y + KH * D, conv_y + 2 * KH * D, C, g, beta, ssm_planes, plane, o, H, KH, M,
                  1.0f / std::sqrt((float)D), false, s, true);
    q27::gated_rmsnorm_q8(o, gnorm_w, z, oxq, oxd, H * M, EPS, s, oxs);
    q27::gdn_flip_plane(plane, s);
    return 0;
  } catch (const std::exception& e) {
    return report(e, err, errlen);
  }
}

// The reference throws std::runtime_error for a bad shape; so must the drop-in (rmsnorm_q8 with n != 5120).
extern "C" int dropin_bad_shape(char* err, int errlen) {
  try {
    q27::rmsnorm_q8(nullptr, nullptr, nullptr, nullptr, nullptr, 4096, 1, EPS, nullptr);
    return 0;
  } catch (const std::runtime_error& e) {
    return report(e, err, errlen);
  }
}

// Prefill of M tokens through an attention layer's fused ops, as src/model.cu's prefill does: embedding gather
// (IQ2_S), attention RMSNorm -> q8_1 (+ h, xs), Q/K norm + RoPE + q8_0 cache write, x += partial with the FFN norm,
// SwiGLU -> q8_1, and the q8_1 quantizer of qmat.h on the attention output.
extern "C" int dropin_attn_prefill(int M, const uint8_t* table, int64_t row_bytes, const int* ids, float* x,
                                   const float* w_attn, float* h, int8_t* xq, float* xd, float* xs, const float* qg,
                                   const float* k, const float* v, const float* qw, const float* kw, float* qn, void* kc,
                                   void* vc, const int* pos0, int n_ctx, float theta_scale, const float* partial,
                                   const float* w_ffn, int8_t* xq2, float* xd2, float* xs2, const float* gate,
                                   const float* up, int ff, int8_t* gq, float* gd, float* gs, const float* ao, int8_t* aq,
                                   float* ad, hipStream_t s, char* err, int errlen) {
  try {
    q27::get_rows_iq2_s(table, row_bytes, ids, M, x, E, s);
    q27::rmsnorm_q8(x, w_attn, h, xq, xd, E, M, EPS, s, xs);
    q27::attn_prep(qg, k, v, qw, kw, qn, kc, vc, pos0, M, EPS, theta_scale, 24, 4, n_ctx, true, s);
    q27::sum_norm_rows(x, partial, E, M, nullptr, w_ffn, EPS, nullptr, xq2, xd2, xs2, s);
    q27::swiglu_q8(gate, up, gq, gd, M * ff, s, gs);
    q27::quantize_q8_1(ao, aq, ad, 6144, M, s);
    return 0;
  } catch (const std::exception& e) {
    return report(e, err, errlen);
  }
}

// Decode GEMV with weights read from a GGUF file: q27::GGUF, qmat_upload (staged transfer + repack), qgemv.
extern "C" int dropin_gguf_gemv(const char* path, const char* name, const int8_t* xq, const float* xd, float* y,
                                int ncols, void* scratch, size_t scratch_bytes, hipStream_t s, char* err, int errlen) {
  try {
    q27::GGUF g(path);
    const q27::GTensor& t = g.tensor(name);
    q27::QMat m = q27::qmat_upload(t, 0, (int)t.ne[1], scratch, scratch_bytes, s);
    q27::qgemv(m, xq, xd, y, ncols, s);
    if (hipStreamSynchronize(s) != hipSuccess) throw std::runtime_error("hipStreamSynchronize failed");
    q27::qmat_free(m);
    return 0;
  } catch (const std::exception& e) {
    return report(e, err, errlen);
  }
}
