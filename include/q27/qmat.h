// Drop-in C++ declaration of the q8_1 activation quantizer of the reference engine's src/qmat.h:50
// (namespace q27; cudaStream_t becomes hipStream_t), forwarding to include/q27h.h.
#pragma once
#include "ops.h"

namespace q27 {

inline void quantize_q8_1(const float* x, int8_t* xq, float* xd, int K, int ncols, hipStream_t s, float* xs = nullptr) {
  q27h_check(q27h_quantize_q8_1(x, xq, xd, K, ncols, s, xs));
}

}  // namespace q27
