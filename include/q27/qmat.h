// Drop-in C++ declarations of the reference engine's src/qmat.h (namespace q27; cudaStream_t becomes hipStream_t):
// the quantized weight matrix QMat, its upload / free, the decode GEMV qgemv and the q8_1 activation quantizer,
// forwarding to include/q27h.h. Bad shapes and unsupported types throw std::runtime_error, as the reference does.
//
// Weight types of qgemv: the ten of the reference (Q2_K, Q4_K, Q6_K, IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ4_XS,
// IQ1_M; q27h_qmat_bytes returns 0 for the others). The prefill
// GEMM (qgemm) and qmat_upload_shard (the two-GPU split) of the reference are not part of this library.
// GType / GTensor come from the drop-in q27/gguf.h (the reference's src/gguf.h).
#pragma once
#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

#include "gguf.h"
#include "ops.h"

namespace q27 {

// src/qmat.h:19-29. `buf` is one device allocation in the tile layout of q27h_qmat_repack; f / d / dw are not used by
// this library (the field offsets follow from type, N and K) and are kept for source compatibility.
struct QMat {
  GType type = GType::F32;
  int N = 0;
  int K = 0;
  int nb = 0;
  int ntiles = 0;
  uint8_t* buf = nullptr;
  size_t bytes = 0;
  uint8_t* f[4] = {nullptr, nullptr, nullptr, nullptr};
  const uint8_t* d = nullptr;
  int dw = 0;
};

// src/qmat.h:31
inline size_t qmat_bytes(GType t, int N, int K) {
  const size_t b = q27h_qmat_bytes((int)t, N, K);
  if (b == 0) throw std::runtime_error("qmat: unsupported type or shape (N % 8, K % 256)");
  return b;
}
// src/qmat.h:42
inline bool qmat_supported(GType t) { return q27h_qmat_bytes((int)t, 8, 256) != 0; }

// The device half of qmat_upload: `raw_dev` holds N GGUF rows ([N][K/256] blocks) in device memory. Allocates the
// matrix buffer (as the reference does) and repacks on stream s.
inline QMat qmat_upload_raw(GType type, int N, int K, const void* raw_dev, hipStream_t s) {
  QMat m;
  m.type = type;
  m.N = N;
  m.K = K;
  m.nb = K / 256;
  m.ntiles = N / 8;
  m.bytes = qmat_bytes(type, N, K);
  if (hipMalloc((void**)&m.buf, m.bytes) != hipSuccess) throw std::runtime_error("qmat: hipMalloc failed");
  const int rc = q27h_qmat_repack((int)type, N, K, raw_dev, m.buf, s);
  if (rc != Q27H_OK) {
    (void)hipFree(m.buf);
    m.buf = nullptr;
    q27h_check(rc);
  }
  return m;
}

// src/qmat.h:34: upload rows [row0, row0 + N) of a GGUF tensor through `scratch` (device, >= N row_bytes) and repack.
// The host -> device transfer is q27h_copy_h2d_staged (pinned staging, several copy threads) instead of one
// cudaMemcpyAsync from the pageable mapping.
inline QMat qmat_upload(const GTensor& t, int row0, int N, void* scratch, size_t scratch_bytes, hipStream_t s) {
  if (row0 < 0 || N < 0 || row0 + N > t.rows()) throw std::runtime_error("qmat: rows outside " + t.name);
  const size_t raw_bytes = (size_t)N * (size_t)t.row_bytes();
  if (raw_bytes > scratch_bytes) throw std::runtime_error("qmat: scratch too small for " + t.name);
  q27h_check(q27h_copy_h2d_staged(scratch, t.data + (size_t)row0 * t.row_bytes(), raw_bytes, 0, s));
  return qmat_upload_raw(t.type, N, (int)t.ne[0], scratch, s);
}

// src/qmat.h:41
inline void qmat_free(QMat& m) {
  if (m.buf) (void)hipFree(m.buf);
  m.buf = nullptr;
}

// src/qmat.h:44-46: y[c][n] = sum_k W[n][k] x[c][k] for c < ncols, x as q8_1 (xq [c][K], xd [c][K/32]).
inline void qgemv(const QMat& m, const int8_t* xq, const float* xd, float* y, int ncols, hipStream_t s) {
  q27h_check(q27h_qgemv((int)m.type, m.N, m.K, m.buf, xq, xd, y, ncols, s));
}

// quantize_q8_1 + qgemv in one launch (no counterpart in the reference; see q27h_qgemv_f32): x f32 [ncols][K].
inline void qgemv_f32(const QMat& m, const float* x, float* y, int ncols, hipStream_t s) {
  q27h_check(q27h_qgemv_f32((int)m.type, m.N, m.K, m.buf, x, y, ncols, s));
}

// src/qmat.h:50
inline void quantize_q8_1(const float* x, int8_t* xq, float* xd, int K, int ncols, hipStream_t s, float* xs = nullptr) {
  q27h_check(q27h_quantize_q8_1(x, xq, xd, K, ncols, s, xs));
}

}  // namespace q27
