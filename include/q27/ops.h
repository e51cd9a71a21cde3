// Drop-in C++ declarations of the fused per-layer ops, with the signatures of the reference engine's src/ops.h
// (namespace q27, same names, parameter order and defaults; cudaStream_t becomes hipStream_t). Each function
// forwards to the C ABI of include/q27h.h and throws std::runtime_error on a non-zero status, as the reference
// launchers throw on bad shapes (src/ops.cu:699,704,724,734) and through CK (src/common.cuh:11-12).
// Declared here: the fused per-layer ops and their unfused twins, the delta-rule recurrence gdn_step and the bf16
// pair GEMV gemv_bf16_pair of src/ops.h. The quantized GEMV is in qmat.h, the prefill row ops in prefill.h; the
// attention kernels of src/ops.h (attn_decode, attn_prefill) are outside this library.
#pragma once
#include <hip/hip_bf16.h>
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstdlib>
#include <stdexcept>
#include <string>

#include "../q27h.h"

namespace q27 {

inline void q27h_check(int status) {
  if (status != Q27H_OK) throw std::runtime_error(std::string("q27h: ") + q27h_last_error());
}

// src/ops.h:15
inline void rmsnorm(const float* x, const float* w, float* y, int n, int rows, float eps, hipStream_t s, int ystride = 0) {
  q27h_check(q27h_rmsnorm(x, w, y, n, rows, eps, s, ystride));
}
// src/ops.h:17
inline void add(const float* x, const float* a, float* y, int n, hipStream_t s) { q27h_check(q27h_add(x, a, y, n, s)); }
// src/ops.h:19
inline void swiglu(const float* g, const float* u, float* y, int n, hipStream_t s) { q27h_check(q27h_swiglu(g, u, y, n, s)); }
// src/ops.h:22-23
inline void get_rows_iq2_s(const uint8_t* table, int64_t row_bytes, const int* ids, int T, float* y, int n, hipStream_t s,
                           const float* img = nullptr) {
  q27h_check(q27h_get_rows_iq2_s(table, row_bytes, ids, T, y, n, s, img));
}
// Same signature for the ggml K-quant / Q8_0 tables (no reference counterpart: its embedding is IQ2_S only).
inline void get_rows_q4_k(const uint8_t* table, int64_t row_bytes, const int* ids, int T, float* y, int n, hipStream_t s,
                          const float* img = nullptr) {
  q27h_check(q27h_get_rows_q4_k(table, row_bytes, ids, T, y, n, s, img));
}
inline void get_rows_q6_k(const uint8_t* table, int64_t row_bytes, const int* ids, int T, float* y, int n, hipStream_t s,
                          const float* img = nullptr) {
  q27h_check(q27h_get_rows_q6_k(table, row_bytes, ids, T, y, n, s, img));
}
inline void get_rows_q8_0(const uint8_t* table, int64_t row_bytes, const int* ids, int T, float* y, int n, hipStream_t s,
                          const float* img = nullptr) {
  q27h_check(q27h_get_rows_q8_0(table, row_bytes, ids, T, y, n, s, img));
}
// src/ops.h:29-30
inline void gdn_gates(const float* a, const float* b, const float* ssm_a, const float* dt_bias, float* g, float* beta, int H,
                      int T, hipStream_t s) {
  q27h_check(q27h_gdn_gates(a, b, ssm_a, dt_bias, g, beta, H, T, s));
}
// src/ops.h:24-26
inline void gemv_bf16_pair(const __hip_bfloat16* Wa, const __hip_bfloat16* Wb, const float* x, float* ya, float* yb, int N,
                           int K, int T, hipStream_t s) {
  q27h_check(q27h_gemv_bf16_pair(reinterpret_cast<const uint16_t*>(Wa), reinterpret_cast<const uint16_t*>(Wb), x, ya, yb, N,
                                 K, T, s));
}
// src/ops.h:32-33
inline void gdn_conv(const float* x, const float* w, float* planes, const int* in_plane, float* y, int C, int T,
                     bool snapshots, hipStream_t s) {
  q27h_check(q27h_gdn_conv(x, w, planes, in_plane, y, C, T, snapshots ? 1 : 0, s));
}
// src/ops.h:40-45. With flip and T >= 128 this runs the chunked form on matrix cores (unless gdn_prefill_exact(true)
// or o overlaps an input): o and the final state then agree with the sequential kernel within float32 rounding
// (relative 1e-5 per 128-value vector), not bit for bit, and T may be at most 65535 * 32.
inline void gdn_step(const float* q, const float* k, const float* v, int stride, const float* g, const float* beta,
                     float* planes, const int* in_plane, float* o, int H, int HK, int T, float scale, bool snapshots,
                     hipStream_t s, bool flip = false) {
  q27h_check(q27h_gdn_step(q, k, v, stride, g, beta, planes, in_plane, o, H, HK, T, scale, snapshots ? 1 : 0, s,
                           flip ? 1 : 0));
}
// No counterpart in the reference: the GDN prefill path bit-exact against the checker (true: gdn_step's prefill
// sequential, gdn_conv_prefill's SiLU and L2 scale correctly rounded) or the faster forms within the 1e-5 fp32 bar
// (false, the default: the chunked recurrence on matrix cores from 128 tokens on, the hardware-exp SiLU and rsq L2
// scale of the conv), process-wide; returns
// the previous setting. Read when a gdn_step call
// enqueues its launch, not at graph replay; threads that change it race with other threads' calls.
inline bool gdn_prefill_exact(bool on) { return q27h_gdn_prefill_exact(on ? 1 : 0) != 0; }
// src/ops.h:36
inline void l2norm_heads(float* x, int n, int heads, int T, int stride, float eps, hipStream_t s) {
  q27h_check(q27h_l2norm_heads(x, n, heads, T, stride, eps, s));
}
// src/ops.h:43
inline void gated_rmsnorm(const float* o, const float* w, const float* z, float* y, int n, int heads, float eps,
                          hipStream_t s) {
  q27h_check(q27h_gated_rmsnorm(o, w, z, y, n, heads, eps, s));
}
// src/ops.h:44
inline void set_int(int* p, int v, hipStream_t s) { q27h_check(q27h_set_int(p, v, s)); }
// src/ops.h:54
inline size_t kv_cache_bytes(int nkvh, int n_ctx, bool q8) { return q27h_kv_cache_bytes(nkvh, n_ctx, q8 ? 1 : 0); }
// src/ops.h:59-62
inline void attn_prep(const float* qg, const float* k, const float* v, const float* q_norm, const float* k_norm, float* qn,
                      void* kcache, void* vcache, const int* pos0, int T, float eps, float theta_scale, int nqh, int nkvh,
                      int n_ctx, bool q8, hipStream_t s, const void* pf = nullptr, size_t pf_bytes = 0,
                      const int* rope3 = nullptr, const int* rdelta = nullptr) {
  q27h_check(q27h_attn_prep(qg, k, v, q_norm, k_norm, qn, kcache, vcache, pos0, T, eps, theta_scale, nqh, nkvh, n_ctx,
                            q8 ? 1 : 0, s, pf, pf_bytes, rope3, rdelta));
}

// src/ops.h:81-97: the two-card exchange arguments. Accepted for source compatibility; a non-null ArArgs* makes
// sum_norm_q8 throw (this library runs one GPU, tensor parallelism is outside it).
struct ArArgs {
  __hip_bfloat16* host_mine = nullptr;
  const __hip_bfloat16* host_other = nullptr;
  int* flag_mine = nullptr;
  const int* flag_other = nullptr;
  const int* dstep = nullptr;
  int n_ar = 0, index = 0;
  int* err = nullptr;
  float* ef = nullptr;
  int ef_first = 1;
  unsigned long long* tprof = nullptr;
};

// src/ops.h:119-120, src/ops.cu:20-30: values per scale on the two-card q8 wire, from Q27_WIRE (read once): "q8" 32,
// "q8b16" 16 (the default), "bf16" 0; anything else throws.
inline int wire_qb() {
  static const int qb = [] {
    const char* e = std::getenv("Q27_WIRE");
    if (!e) return 16;
    const std::string v(e);
    if (v == "q8") return 32;
    if (v == "q8b16") return 16;
    if (v == "bf16") return 0;
    throw std::runtime_error("Q27_WIRE: bf16, q8 or q8b16");
  }();
  return qb;
}
inline bool wire_q8() { return wire_qb() != 0; }

// src/ops.h:99-100
inline void rmsnorm_q8(const float* x, const float* w, float* h, int8_t* xq, float* xd, int n, int rows, float eps,
                       hipStream_t s, float* xs = nullptr) {
  q27h_check(q27h_rmsnorm_q8(x, w, h, xq, xd, n, rows, eps, s, xs));
}
// src/ops.h:103-104
inline void sum_norm_q8(float* x, const float* partial, int n, int rows, const ArArgs* ar, const float* w, float eps, float* h,
                        int8_t* xq, float* xd, hipStream_t s, const void* pf = nullptr, size_t pf_bytes = 0) {
  q27h_check(q27h_sum_norm_q8(x, partial, n, rows, ar, w, eps, h, xq, xd, s, pf, pf_bytes));
}
// src/ops.h:106
inline void swiglu_q8(const float* g, const float* u, int8_t* xq, float* xd, int n, hipStream_t s, float* xs = nullptr) {
  q27h_check(q27h_swiglu_q8(g, u, xq, xd, n, s, xs));
}
// src/ops.h:108-109
inline void gated_rmsnorm_q8(const float* o, const float* w, const float* z, int8_t* xq, float* xd, int heads, float eps,
                             hipStream_t s, float* xs = nullptr) {
  q27h_check(q27h_gated_rmsnorm_q8(o, w, z, xq, xd, heads, eps, s, xs));
}
// src/ops.h:112-114
inline void gdn_conv_l2(const float* x, const float* w, float* planes, const int* in_plane, float* y, int C, int T,
                        bool snapshots, int n_norm_heads, float eps, const float* a, const float* b, const float* ssm_a,
                        const float* dt_bias, float* g, float* beta, int H, hipStream_t s, const void* pf = nullptr,
                        size_t pf_bytes = 0) {
  q27h_check(q27h_gdn_conv_l2(x, w, planes, in_plane, y, C, T, snapshots ? 1 : 0, n_norm_heads, eps, a, b, ssm_a, dt_bias, g,
                              beta, H, s, pf, pf_bytes));
}

}  // namespace q27
