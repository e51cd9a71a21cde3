// Quantized embedding gather: rows of a GGUF-block table (IQ2_S, Q4_K, Q6_K, Q8_0) -> f32 [T][n]; an id < 0
// copies a row of the image-embedding array instead (src/ops.cu:343-375).
//
// One 256-thread workgroup per (token, 5120-value chunk, i.e. one row of the model): the chunk's compressed bytes
// (<= 5440) are first staged in LDS with coalesced dword loads, then each thread decodes groups of 4 consecutive
// values and writes each group as one 16-byte store. Dequantization follows ggml's float order (the reference's IQ2_S kernel and its host
// transcriptions of Q4_K / Q6_K in src/requant.cpp:68-114).
#include "q27h_device.h"
#include "q27h_internal.h"

namespace q27h {
namespace {

__constant__ uint64_t c_iq2s_grid[1024] = {
#include "iq2s_grid.inc"
};

enum Fmt { kIQ2S = 0, kQ4K = 1, kQ6K = 2, kQ80 = 3 };
#ifndef Q27H_ROWS_CHUNK
#define Q27H_ROWS_CHUNK 2560  // half a 5120 row: 9.8 / 10.1 / 10.3 / 9.9 us (Q8_0 / IQ2_S / Q6_K / Q4_K) vs 11.5 / 10.7 / 10.6 / 9.9 for whole rows and 10.7 / 11.3 / 10.5 / 10.3 for 1024
#endif
constexpr int kChunk = Q27H_ROWS_CHUNK;  // values per workgroup

template <int F>
struct FmtInfo;
template <> struct FmtInfo<kIQ2S> { static constexpr int bytes = 82, vals = 256; };
template <> struct FmtInfo<kQ4K> { static constexpr int bytes = 144, vals = 256; };
template <> struct FmtInfo<kQ6K> { static constexpr int bytes = 210, vals = 256; };
template <> struct FmtInfo<kQ80> { static constexpr int bytes = 34, vals = 32; };

__device__ __forceinline__ float h16(const uint8_t* b) { return h2f_bits((uint16_t)(b[0] | (b[1] << 8))); }

template <int F>
__device__ __forceinline__ void decode4(const uint8_t* __restrict__ blk, int r, float (&y)[4]);

// IQ2_S block: d (f16) | qs[32] | signs[32] | qh[8] | scales[8]; value r of the 256 is (ib32, l, j).
template <>
__device__ __forceinline__ void decode4<kIQ2S>(const uint8_t* __restrict__ b, int r, float (&y)[4]) {
  const int ib32 = r >> 5, l = (r >> 3) & 3, j0 = r & 7;
  const float d = h16(b);
  const uint8_t qh = b[66 + ib32], sc = b[74 + ib32];
  const float db = d * (0.5f + (float)((l < 2 ? sc : sc >> 4) & 0xF)) * 0.25f;
  const uint64_t gv = c_iq2s_grid[b[2 + 4 * ib32 + l] | ((qh << (8 - 2 * l)) & 0x300)];
  const uint8_t sg = b[34 + 4 * ib32 + l];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const float g = (float)((gv >> (8 * (j0 + j))) & 0xFF);
    y[j] = db * g * ((sg >> (j0 + j)) & 1 ? -1.f : 1.f);
  }
}

// Q4_K block: d, dmin (f16) | scales[12] | qs[128]; 64-value group j uses scale/min 2j (low nibbles) and 2j+1.
template <>
__device__ __forceinline__ void decode4<kQ4K>(const uint8_t* __restrict__ b, int r, float (&y)[4]) {
  const int jg = r >> 6, hi = (r >> 5) & 1, l0 = r & 31;
  const int is = 2 * jg + hi;
  const uint8_t* q = b + 4;
  uint8_t sc, m;
  if (is < 4) {
    sc = q[is] & 63;
    m = q[is + 4] & 63;
  } else {
    sc = (uint8_t)((q[is + 4] & 0xF) | ((q[is - 4] >> 6) << 4));
    m = (uint8_t)((q[is + 4] >> 4) | ((q[is] >> 6) << 4));
  }
  const float d1 = h16(b) * (float)sc, m1 = h16(b + 2) * (float)m;
  const uint8_t* qs = b + 16 + 32 * jg + l0;
#pragma unroll
  for (int j = 0; j < 4; j++) y[j] = d1 * (float)(hi ? qs[j] >> 4 : qs[j] & 0xF) - m1;
}

// Q6_K block: ql[128] | qh[64] | scales[16] (int8) | d (f16); 128-value halves, quarter qt of a half uses the
// low (qt 0, 1) or high (qt 2, 3) nibbles of ql[l] / ql[l + 32] and bits 2 qt of qh[l].
template <>
__device__ __forceinline__ void decode4<kQ6K>(const uint8_t* __restrict__ b, int r, float (&y)[4]) {
  const int half = r >> 7, qt = (r >> 5) & 3, l0 = r & 31;
  const uint8_t* ql = b + 64 * half + ((qt & 1) ? 32 : 0);
  const uint8_t* qh = b + 128 + 32 * half;
  const int8_t sc = (int8_t)b[192 + 8 * half + (l0 >> 4) + 2 * qt];
  const float d = h16(b + 208);
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int l = l0 + j;
    const int lo = qt < 2 ? (ql[l] & 0xF) : (ql[l] >> 4);
    const int q = (lo | (((qh[l] >> (2 * qt)) & 3) << 4)) - 32;
    y[j] = d * (float)sc * (float)q;
  }
}

// Q8_0 block: d (f16) | qs[32] int8; y = q * d.
template <>
__device__ __forceinline__ void decode4<kQ80>(const uint8_t* __restrict__ b, int r, float (&y)[4]) {
  const float d = h16(b);
#pragma unroll
  for (int j = 0; j < 4; j++) y[j] = (float)(int8_t)b[2 + r + j] * d;
}

#ifndef Q27H_NT_ROWS
#define Q27H_NT_ROWS 1
#endif
constexpr bool kRowsNT = Q27H_NT_ROWS;

template <int F>
__global__ void __launch_bounds__(256) get_rows_kernel(const uint8_t* __restrict__ table, int64_t row_bytes,
                                                       const int* __restrict__ ids, float* __restrict__ y, int n,
                                                       const float* __restrict__ img) {
  constexpr int BB = FmtInfo<F>::bytes, BV = FmtInfo<F>::vals;
  __shared__ uint32_t stage[(kChunk / BV * BB + 3) / 4];
  const int tok = blockIdx.y;
  const int v0 = blockIdx.x * kChunk;
  const int nv = min(kChunk, n - v0);
  const int t = threadIdx.x;
  const int id = ids[tok];
  float* out = y + (size_t)tok * n + v0;
  if (id < 0) {
    for (int o = 4 * t; o < nv; o += 1024) {
      float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
      if (img) a = ld4(img + (size_t)(-id - 1) * n + v0 + o);
      *(float4*)(out + o) = a;
    }
    return;
  }
  const int nblk = (nv + BV - 1) / BV;
  const uint8_t* src = table + (size_t)id * (size_t)row_bytes + (size_t)(v0 / BV) * BB;
  const int nbytes = nblk * BB;
  if ((((uintptr_t)src) & 3) == 0 && (nbytes & 3) == 0) {
    for (int i = t; i < nbytes / 4; i += 256) stage[i] = ((const uint32_t*)src)[i];
  } else {
    uint8_t* sb = (uint8_t*)stage;
    for (int i = t; i < nbytes; i += 256) sb[i] = src[i];
  }
  __syncthreads();
  for (int o = 4 * t; o < nv; o += 1024) {
    float v[4];
    decode4<F>((const uint8_t*)stage + (o / BV) * BB, o % BV, v);
    st4<kRowsNT>(out + o, v[0], v[1], v[2], v[3]);
  }
}

template <int F>
int launch_get_rows(const char* fn, const uint8_t* table, int64_t row_bytes, const int* ids, int T, float* y, int n,
                    q27h_stream_t s, const float* img) {
  constexpr int BV = FmtInfo<F>::vals;
  if (n <= 0 || n % BV || T < 0) return fail(Q27H_ERR_SHAPE, std::string(fn) + ": n must be a positive multiple of " + std::to_string(BV));
  if (row_bytes < (int64_t)(n / BV) * FmtInfo<F>::bytes) return fail(Q27H_ERR_SHAPE, std::string(fn) + ": row_bytes too small");
  if (T == 0) return Q27H_OK;
  if (!table || !ids || !y) return fail(Q27H_ERR_ARG, std::string(fn) + ": null pointer");
  if (!aligned16(y) || (img && !aligned16(img))) return fail(Q27H_ERR_ARG, std::string(fn) + ": y and img need 16-byte alignment");
  if (T > 65535) return fail(Q27H_ERR_SHAPE, std::string(fn) + ": T > 65535");
  hipLaunchKernelGGL(get_rows_kernel<F>, dim3((n + kChunk - 1) / kChunk, T), dim3(256), 0, stream_of(s), table, row_bytes, ids,
                     y, n, img);
  return check_launch(fn);
}

}  // namespace
}  // namespace q27h

using namespace q27h;

extern "C" int q27h_get_rows_iq2_s(const uint8_t* table, int64_t row_bytes, const int* ids, int T, float* y, int n,
                                   q27h_stream_t s, const float* img) {
  return launch_get_rows<kIQ2S>("get_rows_iq2_s", table, row_bytes, ids, T, y, n, s, img);
}
extern "C" int q27h_get_rows_q4_k(const uint8_t* table, int64_t row_bytes, const int* ids, int T, float* y, int n,
                                  q27h_stream_t s, const float* img) {
  return launch_get_rows<kQ4K>("get_rows_q4_k", table, row_bytes, ids, T, y, n, s, img);
}
extern "C" int q27h_get_rows_q6_k(const uint8_t* table, int64_t row_bytes, const int* ids, int T, float* y, int n,
                                  q27h_stream_t s, const float* img) {
  return launch_get_rows<kQ6K>("get_rows_q6_k", table, row_bytes, ids, T, y, n, s, img);
}
extern "C" int q27h_get_rows_q8_0(const uint8_t* table, int64_t row_bytes, const int* ids, int T, float* y, int n,
                                  q27h_stream_t s, const float* img) {
  return launch_get_rows<kQ80>("get_rows_q8_0", table, row_bytes, ids, T, y, n, s, img);
}
