// Host-side plumbing shared by the launchers: status codes, the per-thread error text, launch checks.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "../../include/q27h.h"

namespace q27h {

// Records `msg` as this thread's last error and returns `code`.
int fail(int code, const std::string& msg);
// Checks the launch that was just enqueued; returns Q27H_OK or Q27H_ERR_HIP with the HIP error text.
int check_launch(const char* what);
inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
inline bool aligned4(const void* p) { return ((uintptr_t)p & 3u) == 0; }
inline hipStream_t stream_of(q27h_stream_t s) { return (hipStream_t)s; }
// True when the byte ranges [a, a + na) and [b, b + nb) share a byte.
inline bool overlaps(const void* a, size_t na, const void* b, size_t nb) {
  const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
  return na && nb && x < y + nb && y < x + na;
}

// gdn_rec.hip: whether the process asked for the checker's bits on the GDN prefill path (q27h_gdn_prefill_exact).
bool gdn_prefill_exact_mode();
// gdn_chunk.hip: whether o shares memory with an input of the chunked delta-rule prefill (which it may not).
bool gdn_chunk_o_overlaps(const float* q, const float* k, const float* v, int stride, const float* g, const float* beta,
                          const float* planes, const float* o, int H, int HK, int T);

}  // namespace q27h
