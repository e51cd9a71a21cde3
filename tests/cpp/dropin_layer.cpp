// Test helper: one GDN decode layer and one prefill GDN layer written against the C++ drop-in headers exactly as the
// reference engine's src/model.cu calls them (decode :699-742, prefill :1210-1225), built into a shared library
// that tests/test_gpu_cpp_dropin.py drives through ctypes. It checks that the headers, their default arguments and
// their exceptions work at run time, not only that they compile.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <stdexcept>

#include "q27/ops.h"
#include "q27/prefill.h"

namespace {
constexpr int E = 5120, D = 128, KH = 16, H = 48, C = 2 * KH * D + H * D;
constexpr float EPS = 1e-6f;

int report(const std::exception& e, char* err, int errlen) {
  std::snprintf(err, (size_t)errlen, "%s", e.what());
  return 1;
}
}  // namespace

// Decode, T <= 4 tokens: x += partial, norm -> h and q8_1; conv + l2 + gates with snapshots; the delta rule with
// snapshots; gated norm -> q8_1 of o.
extern "C" int dropin_gdn_decode(int T, float* x, const float* partial, const float* w_norm, float* h, int8_t* xq,
                                 float* xd, const float* conv_in, const float* conv_w, float* conv_planes,
                                 const int* plane, float* conv_y, const float* a, const float* b, const float* ssm_a,
                                 const float* dt_bias, float* g, float* beta, float* ssm_planes, float* o,
                                 const float* gnorm_w, const float* z, int8_t* oxq, float* oxd, hipStream_t s, char* err,
                                 int errlen) {
  try {
    q27::sum_norm_q8(x, partial, E, T, nullptr, w_norm, EPS, h, xq, xd, s);
    q27::gdn_conv_l2(conv_in, conv_w, conv_planes, plane, conv_y, C, T, true, 2 * KH, EPS, a, b, ssm_a, dt_bias, g, beta, H, s);
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
