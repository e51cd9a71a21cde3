// Drop-in C++ declarations of the prefill fused ops, with the signatures of the reference engine's
// src/prefill.h (namespace q27; cudaStream_t becomes hipStream_t), forwarding to include/q27h.h.
#pragma once
#include "ops.h"

namespace q27 {

// src/prefill.h:14-16. y within 4.1e-6 relative (hardware exp2 / rcp / rsq) unless gdn_prefill_exact(true) (q27/ops.h).
inline void gdn_conv_prefill(const float* x, const float* w, float* planes, const int* in_plane, float* y, int C, int M,
                             int n_norm_heads, float eps, const float* a, const float* b, const float* ssm_a,
                             const float* dt_bias, float* g, float* beta, int H, hipStream_t s) {
  q27h_check(q27h_gdn_conv_prefill(x, w, planes, in_plane, y, C, M, n_norm_heads, eps, a, b, ssm_a, dt_bias, g, beta, H, s));
}
// src/prefill.h:18
inline void gdn_flip_plane(int* plane, hipStream_t s) { q27h_check(q27h_gdn_flip_plane(plane, s)); }

// src/prefill.h:21-28: the two-card exchange; a non-null PfExchange* makes sum_norm_rows throw.
struct PfExchange {
  __hip_bfloat16* mine = nullptr;
  const __hip_bfloat16* other = nullptr;
  int* flag_mine = nullptr;
  const int* flag_other = nullptr;
  int token = 0;
  int* err = nullptr;
};

// src/prefill.h:31-32
inline void sum_norm_rows(float* x, const float* partial, int n, int M, const PfExchange* ex, const float* w, float eps,
                          float* h, int8_t* xq, float* xd, float* xs, hipStream_t s) {
  q27h_check(q27h_sum_norm_rows(x, partial, n, M, ex, w, eps, h, xq, xd, xs, s));
}
// src/prefill.h:41
inline void flip_plane_to(int* dst, const int* src, hipStream_t s) { q27h_check(q27h_flip_plane_to(dst, src, s)); }
// src/prefill.h:34-35
inline void to_bf16(const float* x, __hip_bfloat16* y, size_t n, hipStream_t s) {
  q27h_check(q27h_to_bf16(x, reinterpret_cast<uint16_t*>(y), n, s));
}
// src/prefill.h:36-38 (the scale width of the wire is wire_qb(), as in the reference)
inline void to_q8_wire(const float* partial, float* ef, bool first, uint8_t* wire, int n, int M, hipStream_t s) {
  q27h_check(q27h_to_q8_wire(partial, ef, first ? 1 : 0, wire, n, M, wire_qb(), s));
}
// src/prefill.h:39-41
inline void add_norm_rows_q8(float* x, const uint8_t* own, const uint8_t* recv, int n, int M, const float* w, float eps,
                             float* h, int8_t* xq, float* xd, float* xs, hipStream_t s) {
  q27h_check(q27h_add_norm_rows_q8(x, own, recv, n, M, w, eps, h, xq, xd, xs, wire_qb(), s));
}
// src/prefill.h:46-47 (recv = the other card's bf16 partial, or nullptr)
inline void add_norm_rows(float* x, const float* partial, const __hip_bfloat16* recv, int n, int M, const float* w, float eps,
                          float* h, int8_t* xq, float* xd, float* xs, hipStream_t s) {
  q27h_check(q27h_add_norm_rows(x, partial, reinterpret_cast<const uint16_t*>(recv), n, M, w, eps, h, xq, xd, xs, s));
}

}  // namespace q27
