// Decode GEMV over quantized weights (the consumer of the q8_1 activations): y[c][n] = sum_k W[n][k] x[c][k] for
// 1..4 activation columns, W in the ten GGUF block types of the reference (Q2_K, Q4_K, Q6_K, IQ2_XXS, IQ2_XS, IQ2_S,
// IQ3_XXS, IQ3_S, IQ4_XS, IQ1_M) repacked into the tile layout of the
// reference's QMat (src/qmat.h:1-8): 8 rows per tile; chunk = (tile, 256-weight block b, 32-weight sub-block s),
// chunk index (tile * nb + b) * 8 + s; every field of the block struct goes to its own array ordered by chunk, then
// by row inside the tile; the super-block scales go to an array ordered by (tile, block), then row. The repack only
// moves bytes, so every weight decodes to the value it has in the GGUF block.
//
// Kernel (gfx950): one workgroup of W waves per tile (W = 1..16, a function of K only); lane l = 8 lb + s of wave w takes sub-block s of the blocks b = 8 w + lb, + 8 W, ... and keeps the 8 rows x
// ncols partial sums in registers, so one load of its 32 activations per column serves 8 rows. Integer dot products
// per sub-block use v_dot4_i32_i8 (exact); the float contribution of each sub-block is the reference's expression of
// that type (src/qgemv.cu:369-560). The 64 lane sums are added as an xor butterfly in which each exchange level sends
// half of the remaining values (lane xor 32 .. 1), and the W wave sums go through LDS and are added in wave order.
// The same summation order is restated by the CPU checker, so results are bit-identical to it.
#include "q27h_device.h"
#include "q27h_internal.h"

namespace q27h {
namespace {

constexpr int kQ2K = 10, kQ4K = 12, kQ6K = 14, kIQ2XXS = 16, kIQ2XS = 17, kIQ3XXS = 18, kIQ3S = 21, kIQ2S = 22,
              kIQ4XS = 23, kIQ1M = 29;

__device__ const uint32_t kIQ3SGrid[512] = {
#include "iq3s_grid.inc"
};
__device__ const uint32_t kIQ3XXSGrid[256] = {
#include "iq3xxs_grid.inc"
};
__device__ const uint64_t kIQ2XXSGrid[256] = {
#include "iq2xxs_grid.inc"
};
__device__ const uint64_t kIQ2XSGrid[512] = {
#include "iq2xs_grid.inc"
};
__device__ const uint64_t kIQ2SGrid[1024] = {
#include "iq2s_grid.inc"
};
__device__ const uint32_t kIQ1SGrid[2048] = {
#include "iq1s_grid.inc"
};
__device__ const int8_t kIQ4NL[16] = {
#include "iq4nl_values.inc"
};

// Per-type field widths (bytes per chunk, 8 rows), scale bytes per (tile, block), GGUF block bytes.
struct Fmt {
  int nf;
  int w[4];
  int dw;
  int bb;
};
__host__ __device__ constexpr Fmt fmt_of(int type) {
  return type == kQ2K      ? Fmt{2, {64, 16, 0, 0}, 32, 84}
         : type == kQ4K    ? Fmt{2, {128, 16, 0, 0}, 32, 144}
         : type == kQ6K    ? Fmt{3, {128, 64, 16, 0}, 16, 210}
         : type == kIQ2XXS ? Fmt{1, {64, 0, 0, 0}, 16, 66}
         : type == kIQ2XS  ? Fmt{2, {64, 8, 0, 0}, 16, 74}
         : type == kIQ3XXS ? Fmt{2, {64, 32, 0, 0}, 16, 98}
         : type == kIQ3S   ? Fmt{4, {64, 32, 8, 4}, 16, 110}
         : type == kIQ2S   ? Fmt{4, {32, 32, 8, 8}, 16, 82}
         : type == kIQ4XS  ? Fmt{2, {128, 8, 0, 0}, 16, 136}
         : type == kIQ1M   ? Fmt{3, {32, 16, 8, 0}, 16, 56}
                           : Fmt{0, {0, 0, 0, 0}, 0, 0};
}
inline size_t align256(size_t x) { return (x + 255) / 256 * 256; }

struct Mat {
  const uint8_t* f[4];
  const uint8_t* d;
  int N, nb, ntiles;
};

// Where the bytes of a chunk's field go. Fields of up to 16 bytes per chunk are stored chunk after chunk (chunk
// index (tile * nb + b) * 8 + s), so the 32 chunks of 4 consecutive blocks are contiguous. Wider fields are cut in
// 16-byte pieces and, per tile, per group of 4 blocks, piece i of the group's 32 chunks lies together: one 16-byte
// load per lane of a half-wave (4 blocks x 8 sub-blocks) then reads 512 contiguous bytes. A tile's block count is
// padded to a multiple of 4 for these fields.
__host__ __device__ __forceinline__ size_t field_off(int wf, size_t tile, int nb, int b, int s) {
  if (wf <= 16) return ((tile * nb + b) * 8 + s) * wf;
  const size_t g = tile * ((nb + 3) / 4) + b / 4;
  return (g * (wf / 16) * 32 + (b % 4) * 8 + s) * 16;  // + piece i at i * 512
}
__host__ __device__ constexpr size_t field_bytes(int wf, size_t ntiles, int nb) {
  return wf <= 16 ? ntiles * nb * 8 * wf : ntiles * ((nb + 3) / 4) * 32 * wf;
}

// Field offsets inside the QMat buffer: the fields in order, then the scales, each 256-byte aligned.
size_t layout(int type, int N, int K, size_t off[5]) {
  const Fmt F = fmt_of(type);
  const size_t ntiles = N / 8;
  const int nb = K / 256;
  size_t o = 0;
  for (int i = 0; i < 4; i++) {
    off[i] = o;
    if (i < F.nf) o += align256(field_bytes(F.w[i], ntiles, nb));
  }
  off[4] = o;
  return o + align256(ntiles * nb * F.dw);
}

// ---------------------------------------------------------------- repack (one workgroup per tile and group of 4 blocks)
// The 8 rows x (up to) 4 GGUF blocks of a group are read into LDS with coalesced 4-byte loads; thread t = 8 c + r
// (chunk c = 8 bl + s of the group, row r) builds row r's part of chunk c's record (every field of a chunk record is
// row-major: W = wf / 8 bytes per row) into an LDS image of the destination, which is then written with 16-byte
// stores. A group covers exactly the 32 chunks of one group of the wide (16-byte piece) fields, so its image of such a
// field is one contiguous 32 x wf-byte range; the narrow fields and the scales of the group's blocks are contiguous
// too. Chunks of a tail group past the row's last block are padding of the wide fields and are written as zeros.
constexpr int kRepackBlocks = 4;

// Writes the W bytes v (row r of chunk c) to their place in the group image of a field of wf bytes per chunk.
template <int WF, int W>
__device__ __forceinline__ void put_row(uint8_t* img, int c, int r, const uint8_t (&v)[W], uint32_t keep) {
  const int j0 = W * r;
  uint8_t* d = img + (WF <= 16 ? c * WF + j0 : (j0 / 16) * 512 + c * 16 + j0 % 16);
  if constexpr (W % 4 == 0) {
#pragma unroll
    for (int k = 0; k < W / 4; k++)
      ((uint32_t*)d)[k] = ((uint32_t)v[4 * k] | ((uint32_t)v[4 * k + 1] << 8) | ((uint32_t)v[4 * k + 2] << 16) |
                           ((uint32_t)v[4 * k + 3] << 24)) & keep;
  } else if constexpr (W == 2) {
    *(uint16_t*)d = (uint16_t)(((uint32_t)v[0] | ((uint32_t)v[1] << 8)) & keep);
  } else {
    *d = (uint8_t)(v[0] & keep);
  }
}

// Copies n bytes (a multiple of 16) of an LDS image to dst (16-byte aligned).
__device__ __forceinline__ void copy_out(uint8_t* __restrict__ dst, const uint8_t* img, int n) {
  for (int u = threadIdx.x; u < n / 16; u += 256) ((uint4*)dst)[u] = ((const uint4*)img)[u];
}

template <int TYPE>
__global__ void __launch_bounds__(256) repack_kernel(const uint8_t* __restrict__ raw, uint8_t* __restrict__ f0,
                                                     uint8_t* __restrict__ f1, uint8_t* __restrict__ f2,
                                                     uint8_t* __restrict__ f3, uint8_t* __restrict__ dd, int nb) {
  constexpr Fmt F = fmt_of(TYPE);
  constexpr int RS = kRepackBlocks * F.bb;  // LDS bytes per row
  __shared__ __align__(16) uint8_t sraw[8 * RS];
  __shared__ __align__(16) uint8_t img0[32 * F.w[0]];
  __shared__ __align__(16) uint8_t img1[32 * (F.w[1] ? F.w[1] : 16)];
  __shared__ __align__(16) uint8_t img2[32 * (F.w[2] ? F.w[2] : 16)];
  __shared__ __align__(16) uint8_t img3[32 * (F.w[3] ? F.w[3] : 16)];
  __shared__ __align__(16) uint8_t imgd[kRepackBlocks * F.dw];
  const int ngroups = (nb + kRepackBlocks - 1) / kRepackBlocks;
  const size_t tile = blockIdx.x / ngroups;
  const int g = (int)(blockIdx.x % ngroups);
  const int b0 = g * kRepackBlocks;
  const int nbg = min(kRepackBlocks, nb - b0);
  const int t = threadIdx.x;

  // raw rows of the group -> LDS (row r at r * RS): 32 lanes per row, 4-byte loads when every row starts at a
  // multiple of 4 bytes (the group's start in its row, 4 g blocks, always does), else 2-byte loads (GGUF blocks have
  // even sizes), or bytes for an odd raw pointer
  const int L = nbg * F.bb;
  {
    const int rr = t >> 5, k0 = t & 31;
    const uint8_t* row = raw + ((tile * 8 + rr) * nb + b0) * F.bb;
    uint8_t* lrow = sraw + rr * RS;
    if ((((uintptr_t)raw | ((size_t)nb * F.bb)) & 3) == 0) {
      for (int k = k0; k < L / 4; k += 32)
        ((uint32_t*)lrow)[k] = __builtin_nontemporal_load((const uint32_t*)row + k);
      if ((L & 2) && k0 == 0) ((uint16_t*)lrow)[L / 2 - 1] = __builtin_nontemporal_load((const uint16_t*)row + L / 2 - 1);
    } else if (((uintptr_t)raw & 1) == 0) {
      for (int k = k0; k < L / 2; k += 32)
        ((uint16_t*)lrow)[k] = __builtin_nontemporal_load((const uint16_t*)row + k);
    } else {
      for (int k = k0; k < L; k += 32) lrow[k] = row[k];
    }
  }
  __syncthreads();

  const int c = t >> 3, r = t & 7, bl = c >> 3, s = c & 7;
  const uint32_t keep = bl < nbg ? ~0u : 0u;
  const uint8_t* src = sraw + r * RS + (bl < nbg ? bl : 0) * F.bb;
  uint8_t* od = imgd + bl * F.dw;
  const bool put_d = s == 0 && bl < nbg;
  if constexpr (TYPE == kQ4K) {  // d, dmin, scales[12], qs[128]
    const uint8_t* qs = src + 16 + 32 * (s / 2);
    const int sh = 4 * (s & 1);
    uint8_t o0[16], o1[2];
#pragma unroll
    for (int k = 0; k < 16; k++)  // byte k: weight k (low nibble), weight k + 16 (high nibble)
      o0[k] = (uint8_t)(((qs[k] >> sh) & 0xF) | (((qs[k + 16] >> sh) & 0xF) << 4));
    const uint8_t* sc = src + 4;
    int scv, mv;
    if (s < 4) {
      scv = sc[s] & 63;
      mv = sc[s + 4] & 63;
    } else {
      scv = (sc[s + 4] & 0xF) | ((sc[s - 4] >> 6) << 4);
      mv = (sc[s + 4] >> 4) | ((sc[s] >> 6) << 4);
    }
    o1[0] = (uint8_t)scv;
    o1[1] = (uint8_t)mv;
    put_row<F.w[0]>(img0, c, r, o0, keep);
    put_row<F.w[1]>(img1, c, r, o1, keep);
    if (put_d)
      for (int k = 0; k < 4; k++) od[4 * r + k] = src[k];
  } else if constexpr (TYPE == kQ6K) {  // ql[128], qh[64], scales[16], d
    const int n = s / 4, j = s % 4;
    uint8_t q[32], o0[16], o1[8], o2[2];
#pragma unroll
    for (int l = 0; l < 32; l++) {
      const uint8_t lo = src[64 * n + 32 * (j & 1) + l];
      const uint8_t hi = src[128 + 32 * n + l];
      q[l] = (uint8_t)(((j < 2 ? lo : lo >> 4) & 0xF) | (((hi >> (2 * j)) & 3) << 4));
    }
#pragma unroll
    for (int k = 0; k < 16; k++) o0[k] = (uint8_t)((q[k] & 0xF) | ((q[k + 16] & 0xF) << 4));
#pragma unroll
    for (int h = 0; h < 2; h++)  // word h (weights 16 h ..): byte k holds the high bits of weights 16 h + k + 4 i
#pragma unroll
      for (int k = 0; k < 4; k++) {
        uint8_t v = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) v |= (uint8_t)(((q[16 * h + k + 4 * i] >> 4) & 3) << (2 * i));
        o1[4 * h + k] = v;
      }
    o2[0] = src[192 + 8 * n + 2 * j];
    o2[1] = src[192 + 8 * n + 2 * j + 1];
    put_row<F.w[0]>(img0, c, r, o0, keep);
    put_row<F.w[1]>(img1, c, r, o1, keep);
    put_row<F.w[2]>(img2, c, r, o2, keep);
    if (put_d) {
      od[2 * r] = src[208];
      od[2 * r + 1] = src[209];
    }
  } else if constexpr (TYPE == kIQ3S) {  // d, qs[64], qh[8], signs[32], scales[4]
    uint8_t o0[8], o1[4], o2[1];
#pragma unroll
    for (int k = 0; k < 8; k++) o0[k] = src[2 + 8 * s + k];
#pragma unroll
    for (int k = 0; k < 4; k++) o1[k] = src[74 + 4 * s + k];
    o2[0] = src[66 + s];
    put_row<F.w[0]>(img0, c, r, o0, keep);
    put_row<F.w[1]>(img1, c, r, o1, keep);
    put_row<F.w[2]>(img2, c, r, o2, keep);
    // the scale nibbles of the chunk's 8 rows in one word (row r at bits 4 r): byte r / 2 from rows r, r + 1
    const uint32_t nib = (src[106 + s / 2] >> (4 * (s & 1))) & 0xF;
    const uint32_t next = (uint32_t)__shfl_down((int)nib, 1);
    if (!(r & 1)) img3[4 * c + r / 2] = (uint8_t)((nib | (next << 4)) & keep);
    if (put_d) {
      od[2 * r] = src[0];
      od[2 * r + 1] = src[1];
    }
  } else if constexpr (TYPE == kIQ4XS) {  // d, scales_h (u16), scales_l[4], qs[128]
    uint8_t o0[16], o1[1];
#pragma unroll
    for (int k = 0; k < 16; k++) o0[k] = src[8 + 16 * s + k];
    const int sh = src[2] | (src[3] << 8);
    const int l = ((src[4 + s / 2] >> (4 * (s & 1))) & 0xF) | (((sh >> (2 * s)) & 3) << 4);
    o1[0] = (uint8_t)(int8_t)(l - 32);
    put_row<F.w[0]>(img0, c, r, o0, keep);
    put_row<F.w[1]>(img1, c, r, o1, keep);
    if (put_d) {
      od[2 * r] = src[0];
      od[2 * r + 1] = src[1];
    }
  } else if constexpr (TYPE == kQ2K) {  // scales[16], qs[64], d, dmin
    // sub-block s = 4 n + j: weights 128 n + 32 j + l = (qs[32 n + l] >> 2 j) & 3. Word h (weights 16 h ..):
    // byte k holds weights 16 h + k + 4 i at bits 2 i.
    const int n = s / 4, j = s % 4;
    const uint8_t* qs = src + 16 + 32 * n;
    uint8_t o0[8], o1[2];
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
      for (int k = 0; k < 4; k++) {
        uint8_t v = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) v |= (uint8_t)(((qs[16 * h + k + 4 * i] >> (2 * j)) & 3) << (2 * i));
        o0[4 * h + k] = v;
      }
    o1[0] = src[8 * n + 2 * j];
    o1[1] = src[8 * n + 2 * j + 1];
    put_row<F.w[0]>(img0, c, r, o0, keep);
    put_row<F.w[1]>(img1, c, r, o1, keep);
    if (put_d)
      for (int k = 0; k < 4; k++) od[4 * r + k] = src[80 + k];
  } else if constexpr (TYPE == kIQ2XXS) {  // d, per sub-block 4 grid indices + a sign / scale word
    uint8_t o0[8];
#pragma unroll
    for (int k = 0; k < 8; k++) o0[k] = src[2 + 8 * s + k];
    put_row<F.w[0]>(img0, c, r, o0, keep);
    if (put_d) {
      od[2 * r] = src[0];
      od[2 * r + 1] = src[1];
    }
  } else if constexpr (TYPE == kIQ2XS) {  // d, qs[32] (u16 index + signs), scales[8]
    uint8_t o0[8], o1[1];
#pragma unroll
    for (int k = 0; k < 8; k++) o0[k] = src[2 + 8 * s + k];
    o1[0] = src[66 + s];
    put_row<F.w[0]>(img0, c, r, o0, keep);
    put_row<F.w[1]>(img1, c, r, o1, keep);
    if (put_d) {
      od[2 * r] = src[0];
      od[2 * r + 1] = src[1];
    }
  } else if constexpr (TYPE == kIQ3XXS) {  // d, qs[64], scales_and_signs[32]
    uint8_t o0[8], o1[4];
#pragma unroll
    for (int k = 0; k < 8; k++) o0[k] = src[2 + 8 * s + k];
#pragma unroll
    for (int k = 0; k < 4; k++) o1[k] = src[66 + 4 * s + k];
    put_row<F.w[0]>(img0, c, r, o0, keep);
    put_row<F.w[1]>(img1, c, r, o1, keep);
    if (put_d) {
      od[2 * r] = src[0];
      od[2 * r + 1] = src[1];
    }
  } else if constexpr (TYPE == kIQ2S) {  // d, qs[32], signs[32], qh[8], scales[8]
    uint8_t o0[4], o1[4], o2[1], o3[1];
#pragma unroll
    for (int k = 0; k < 4; k++) o0[k] = src[2 + 4 * s + k];
#pragma unroll
    for (int k = 0; k < 4; k++) o1[k] = src[34 + 4 * s + k];
    o2[0] = src[66 + s];
    o3[0] = src[74 + s];
    put_row<F.w[0]>(img0, c, r, o0, keep);
    put_row<F.w[1]>(img1, c, r, o1, keep);
    put_row<F.w[2]>(img2, c, r, o2, keep);
    put_row<F.w[3]>(img3, c, r, o3, keep);
    if (put_d) {
      od[2 * r] = src[0];
      od[2 * r + 1] = src[1];
    }
  } else if constexpr (TYPE == kIQ1M) {  // qs[32], qh[16], scales[8] (4 x u16, fp16 scale in the top nibbles)
    uint8_t o0[4], o1[2], o2[1];
#pragma unroll
    for (int k = 0; k < 4; k++) o0[k] = src[4 * s + k];
    o1[0] = src[32 + 2 * s];
    o1[1] = src[33 + 2 * s];
    uint16_t s16[4];
#pragma unroll
    for (int k = 0; k < 4; k++) s16[k] = (uint16_t)(src[48 + 2 * k] | (src[49 + 2 * k] << 8));
    o2[0] = (uint8_t)((s16[s / 2] >> (6 * (s % 2))) & 63);
    put_row<F.w[0]>(img0, c, r, o0, keep);
    put_row<F.w[1]>(img1, c, r, o1, keep);
    put_row<F.w[2]>(img2, c, r, o2, keep);
    if (put_d) {
      const uint16_t dh = (uint16_t)((s16[0] >> 12) | ((s16[1] >> 8) & 0x00F0) | ((s16[2] >> 4) & 0x0F00) | (s16[3] & 0xF000));
      od[2 * r] = (uint8_t)(dh & 0xFF);
      od[2 * r + 1] = (uint8_t)(dh >> 8);
    }
  }
  __syncthreads();

  // images -> the fields: wide fields as the group's whole 32 x wf range, narrow ones and the scales for nbg blocks
  const size_t tb0 = tile * nb + b0;
  auto out = [&](uint8_t* f, int wf, const uint8_t* img) {
    if (wf > 16) copy_out(f + (tile * ngroups + g) * 32 * (size_t)wf, img, 32 * wf);
    else copy_out(f + tb0 * 8 * wf, img, nbg * 8 * wf);
  };
  out(f0, F.w[0], img0);
  if constexpr (F.nf > 1) out(f1, F.w[1], img1);
  if constexpr (F.nf > 2) out(f2, F.w[2], img2);
  if constexpr (F.nf > 3) out(f3, F.w[3], img3);
  copy_out(dd + tb0 * F.dw, imgd, nbg * F.dw);
}
// ---------------------------------------------------------------- decode of one chunk
__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }
// Exact integer product of operands within 24 bits whose product fits 32 bits (v_mul_i32_i24, full rate; a plain
// 32-bit multiply is a quarter-rate instruction). Every product below satisfies both bounds: |sum of a sub-block| <
// 2^19 and |scale| < 2^7.
__device__ __forceinline__ int mul24(int a, int b) { return ((a << 8) >> 8) * ((b << 8) >> 8); }
__device__ __forceinline__ float half_lo(uint32_t w) { return h2f_bits((uint16_t)(w & 0xFFFF)); }
__device__ __forceinline__ float half_hi(uint32_t w) { return h2f_bits((uint16_t)(w >> 16)); }
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
// Cache policy of the weight loads. The small per-chunk fields and scales: nontemporal (SMALL). The wide
// interleaved pieces: chosen per launch from K (kNtPiecesMaxK): nontemporal for K <= 8192 (many tiles of short rows),
// ordinary loads beyond. Measured (us, T = 1, nontemporal / ordinary pieces): 5120 x 17408 Q6_K 17.9 / 16.6, Q4_K
// 14.4 / 13.8, IQ4_XS 15.9 / 15.0, Q2_K 11.1 / 10.6; 17408 x 5120 Q6_K 14.6 / 15.2, Q4_K 11.0 / 11.4, IQ4_XS 12.1 /
// 12.7. rocprofv3 FETCH_SIZE shows why: with nontemporal pieces a 5120 x 17408 Q6_K launch fetches 98 MB for its
// 73 MB matrix, with ordinary loads 75-77 MB.
constexpr int kNtPiecesMaxK = 8192;
#ifndef Q27H_QG_NT_SMALL
#define Q27H_QG_NT_SMALL 1
#endif
template <int N, bool NT = Q27H_QG_NT_SMALL>
__device__ __forceinline__ void ld16(uint32_t* w, const uint8_t* p) {  // N x 16 bytes, read once
#pragma unroll
  for (int i = 0; i < N; i++) {
    u32x4 v;
    if constexpr (NT) v = __builtin_nontemporal_load((const u32x4*)p + i);
    else v = ((const u32x4*)p)[i];
    w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
  }
}

// IQ4_XS levels of 4 nibbles (one per byte, values 0..15) via two byte permutes of the 16-entry table.
__device__ __forceinline__ int iq4_levels(uint32_t nib, const uint32_t (&t)[4]) {
  const uint32_t sel = nib & 0x07070707u;
  const uint32_t lo = __builtin_amdgcn_perm(t[1], t[0], sel);  // entries 0..7
  const uint32_t hi = __builtin_amdgcn_perm(t[3], t[2], sel);  // entries 8..15
  const uint32_t m = ((nib >> 3) & 0x01010101u) * 0xFFu;
  return (int)((hi & m) | (lo & ~m));
}

// Tables of a type in LDS: `grid` words of codebook, then `masks` entries of two words (the 0x00 / 0xFF byte masks
// of the low and high nibble of a sign byte; 128 entries = ksigns of 7 bits, 256 = the byte itself).
template <int TYPE>
struct LutInfo {
  static constexpr int grid = TYPE == kIQ3S ? 512 : TYPE == kIQ2XXS ? 512 : TYPE == kIQ2XS ? 1024 : TYPE == kIQ2S ? 2048
                              : TYPE == kIQ3XXS ? 256 : TYPE == kIQ1M ? 2048 : 0;
  static constexpr int masks = TYPE == kIQ3S || TYPE == kIQ2S ? 256 : TYPE == kIQ2XXS || TYPE == kIQ2XS || TYPE == kIQ3XXS ? 128 : 0;
  static constexpr int words = grid + 2 * masks;
};

template <int TYPE>
struct Chunk {
  static constexpr Fmt F = fmt_of(TYPE);
  static constexpr int nw = (F.w[0] + F.w[1] + F.w[2] + F.w[3]) / 4 + F.dw / 4;
  uint32_t w[nw];
};

// N 16-byte pieces of a field wider than 16 bytes (pieces 512 bytes apart, see field_off)
template <int N, bool NTP>
__device__ __forceinline__ void ldp_(uint32_t* w, const uint8_t* p) {
#pragma unroll
  for (int i = 0; i < N; i++) ld16<1, NTP>(w + 4 * i, p + 512 * i);
}

template <int TYPE, bool NTP>
__device__ __forceinline__ void load_chunk(Chunk<TYPE>& c, const Mat& m, size_t tile, int b, int s) {
  const size_t tb = tile * m.nb + b;
  if constexpr (TYPE == kQ4K) {
    ldp_<8, NTP>(c.w, m.f[0] + field_off(128, tile, m.nb, b, s));
    ld16<1>(c.w + 32, m.f[1] + field_off(16, tile, m.nb, b, s));
    ld16<2>(c.w + 36, m.d + tb * 32);
  } else if constexpr (TYPE == kQ6K) {
    ldp_<8, NTP>(c.w, m.f[0] + field_off(128, tile, m.nb, b, s));
    ldp_<4, NTP>(c.w + 32, m.f[1] + field_off(64, tile, m.nb, b, s));
    ld16<1>(c.w + 48, m.f[2] + field_off(16, tile, m.nb, b, s));
    ld16<1>(c.w + 52, m.d + tb * 16);
  } else if constexpr (TYPE == kIQ3S) {
    ldp_<4, NTP>(c.w, m.f[0] + field_off(64, tile, m.nb, b, s));
    ldp_<2, NTP>(c.w + 16, m.f[1] + field_off(32, tile, m.nb, b, s));
    const u32x2 h = *(const u32x2*)(m.f[2] + field_off(8, tile, m.nb, b, s));
    c.w[24] = h.x; c.w[25] = h.y;
    c.w[26] = *(const uint32_t*)(m.f[3] + field_off(4, tile, m.nb, b, s));
    ld16<1>(c.w + 27, m.d + tb * 16);
  } else if constexpr (TYPE == kIQ4XS) {
    ldp_<8, NTP>(c.w, m.f[0] + field_off(128, tile, m.nb, b, s));
    const u32x2 l = *(const u32x2*)(m.f[1] + field_off(8, tile, m.nb, b, s));
    c.w[32] = l.x; c.w[33] = l.y;
    ld16<1>(c.w + 34, m.d + tb * 16);
  } else if constexpr (TYPE == kQ2K) {
    ldp_<4, NTP>(c.w, m.f[0] + field_off(64, tile, m.nb, b, s));
    ld16<1>(c.w + 16, m.f[1] + field_off(16, tile, m.nb, b, s));
    ld16<2>(c.w + 20, m.d + tb * 32);
  } else if constexpr (TYPE == kIQ2XXS) {
    ldp_<4, NTP>(c.w, m.f[0] + field_off(64, tile, m.nb, b, s));
    ld16<1>(c.w + 16, m.d + tb * 16);
  } else if constexpr (TYPE == kIQ2XS) {
    ldp_<4, NTP>(c.w, m.f[0] + field_off(64, tile, m.nb, b, s));
    const u32x2 l = *(const u32x2*)(m.f[1] + field_off(8, tile, m.nb, b, s));
    c.w[16] = l.x; c.w[17] = l.y;
    ld16<1>(c.w + 18, m.d + tb * 16);
  } else if constexpr (TYPE == kIQ3XXS) {
    ldp_<4, NTP>(c.w, m.f[0] + field_off(64, tile, m.nb, b, s));
    ldp_<2, NTP>(c.w + 16, m.f[1] + field_off(32, tile, m.nb, b, s));
    ld16<1>(c.w + 24, m.d + tb * 16);
  } else if constexpr (TYPE == kIQ2S) {
    ldp_<2, NTP>(c.w, m.f[0] + field_off(32, tile, m.nb, b, s));
    ldp_<2, NTP>(c.w + 8, m.f[1] + field_off(32, tile, m.nb, b, s));
    const u32x2 h = *(const u32x2*)(m.f[2] + field_off(8, tile, m.nb, b, s));
    c.w[16] = h.x; c.w[17] = h.y;
    const u32x2 l = *(const u32x2*)(m.f[3] + field_off(8, tile, m.nb, b, s));
    c.w[18] = l.x; c.w[19] = l.y;
    ld16<1>(c.w + 20, m.d + tb * 16);
  } else if constexpr (TYPE == kIQ1M) {
    ldp_<2, NTP>(c.w, m.f[0] + field_off(32, tile, m.nb, b, s));
    ld16<1>(c.w + 8, m.f[1] + field_off(16, tile, m.nb, b, s));
    const u32x2 l = *(const u32x2*)(m.f[2] + field_off(8, tile, m.nb, b, s));
    c.w[12] = l.x; c.w[13] = l.y;
    ld16<1>(c.w + 14, m.d + tb * 16);
  }
}

// Types whose four-column, one-block-per-lane kernel parks the sums of rows 0-3 in LDS (dot_chunk's PARK). Measured
// (us, 17408 x 5120 / 6144 x 5120, T = 4, against the sums in registers): IQ3_S 18.9 / 9.9-10.0 against 19.7-19.8 /
// 10.1 (and no scratch), IQ2_XXS 18.3-18.6 / 9.3-9.5 against 18.9 / 9.6, IQ1_M 22.1-22.2 / 11.75 against 22.8-22.9 /
// 11.8; Q6_K (21.2-21.5 against 20.0) and IQ4_XS (18.0 against 17.6) ran slower, Q2_K, IQ2_XS, IQ3_XXS and IQ2_S the
// same within noise.
constexpr bool parks_sums(int type) { return type == kIQ3S || type == kIQ2XXS || type == kIQ1M; }

// acc[r * NC + c] += t, or with PARK and r < 4 the finished sum to the lane's LDS slot (see dot_chunk).
template <bool PARK, int NC>
__device__ __forceinline__ void acc_add(float (&acc)[8 * NC], float* park, int r, int c, float t) {
  if constexpr (PARK) {
    if (r < 4) {
      park[(r * NC + c) * 256] = acc[r * NC + c] + t;
      return;
    }
  }
  acc[r * NC + c] += t;
}

// acc[r * NC + c] += t(row r, column c) for one chunk; u[c] = the 32 int8 activations of column c, dy[c] its scale.
// PARK: the sums of rows 0-3 go to LDS (park[value * 256], the lane's own slots) as soon as the row is done, instead
// of staying in registers for the whole chunk; used where a lane has one chunk, so the parked value is the
// accumulator's final one.
template <int TYPE, int NC, bool PARK = false>
__device__ __forceinline__ void dot_chunk(const Chunk<TYPE>& ch, const int (&u)[NC][8], const float (&dy)[NC],
                                          const uint32_t* __restrict__ lut, const uint32_t (&kv)[4],
                                          float (&acc)[8 * NC], float* park = nullptr) {
  const uint32_t* w = ch.w;
  if constexpr (TYPE == kQ4K) {
    // (the min term's (float)(s8 * m) equals (float)s8 * (float)m exactly, |s8 * m| < 2^24; that form, one multiply
    // instead of a 24-bit multiply and a conversion per row and column, measured slower: 5120 x 17408 T = 4 20.3
    // against 18.8 us)
    int s8[NC];  // sums of the activations: the min term (dmin * m) multiplies them
#pragma unroll
    for (int c = 0; c < NC; c++) {
      int t = 0;
#pragma unroll
      for (int k = 0; k < 8; k++) t = dot4(u[c][k], 0x01010101, t);
      s8[c] = t;
    }
#pragma unroll
    for (int r = 0; r < 8; r++) {
      int sumi[NC];
#pragma unroll
      for (int c = 0; c < NC; c++) sumi[c] = 0;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int lo = (int)(w[4 * r + j] & 0x0F0F0F0Fu), hi = (int)((w[4 * r + j] >> 4) & 0x0F0F0F0Fu);
#pragma unroll
        for (int c = 0; c < NC; c++) sumi[c] = dot4(hi, u[c][j + 4], dot4(lo, u[c][j], sumi[c]));
      }
      const uint32_t sm = w[32 + r / 2] >> (16 * (r & 1));
      const int sc = (int)(sm & 0xFF), mn = (int)((sm >> 8) & 0xFF);
      const float d = half_lo(w[36 + r]), dmin = half_hi(w[36 + r]);
#pragma unroll
      for (int c = 0; c < NC; c++)
        acc_add<PARK, NC>(acc, park, r, c,
                          d * (dy[c] * (float)mul24(sumi[c], sc)) - dmin * (dy[c] * (float)mul24(s8[c], mn)));
    }
  } else if constexpr (TYPE == kQ6K) {
    int s8a[NC], s8b[NC];  // activation sums of the two 16-weight halves (the -32 offset of the quants)
#pragma unroll
    for (int c = 0; c < NC; c++) {
      int ta = 0, tb = 0;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        ta = dot4(u[c][k], 0x01010101, ta);
        tb = dot4(u[c][k + 4], 0x01010101, tb);
      }
      s8a[c] = ta;
      s8b[c] = tb;
    }
#pragma unroll
    for (int r = 0; r < 8; r++) {
      int sa[NC], sb[NC];
#pragma unroll
      for (int c = 0; c < NC; c++) sa[c] = sb[c] = 0;
      const uint32_t h0 = w[32 + 2 * r], h1 = w[33 + 2 * r];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t l = w[4 * r + i];
        const int qa = (int)((l & 0x0F0F0F0Fu) | (((h0 >> (2 * i)) & 0x03030303u) << 4));
        const int qb = (int)(((l >> 4) & 0x0F0F0F0Fu) | (((h1 >> (2 * i)) & 0x03030303u) << 4));
#pragma unroll
        for (int c = 0; c < NC; c++) {
          sa[c] = dot4(qa, u[c][i], sa[c]);
          sb[c] = dot4(qb, u[c][4 + i], sb[c]);
        }
      }
      const uint32_t g = w[48 + r / 2] >> (16 * (r & 1));
      const int sc0 = (int)(int8_t)(g & 0xFF), sc1 = (int)(int8_t)((g >> 8) & 0xFF);
      const float d = (r & 1) ? half_hi(w[52 + r / 2]) : half_lo(w[52 + r / 2]);
#pragma unroll
      for (int c = 0; c < NC; c++) {
        const int si = mul24(sa[c] - 32 * s8a[c], sc0) + mul24(sb[c] - 32 * s8b[c], sc1);
        acc_add<PARK, NC>(acc, park, r, c, d * (dy[c] * (float)si));
      }
    }
  } else if constexpr (TYPE == kIQ3S) {
    // lut[0..511] = the codebook, lut[512..1023] = per sign byte the byte masks (0x00 / 0xFF) of its two nibbles
    const uint2* smask = (const uint2*)(lut + LutInfo<TYPE>::grid);
#pragma unroll
    for (int r = 0; r < 8; r++) {
      const uint32_t qh = (w[24 + r / 4] >> (8 * (r & 3))) & 0xFF;
      const uint32_t sg = w[16 + r];
      // all 12 table reads of the row first, then the arithmetic: one LDS wait per row instead of one per lookup
      uint32_t g[8];
      uint2 mm[4];
      if constexpr (NC < 4 || PARK) {
        // 9-bit index k = qs byte k | qh bit k << 8, assembled by one byte permute from the qs word and the qh bits
        // spread to bytes (byte j of hb[h] = bit 4 h + j of qh). The prefetching four-column kernel, which keeps all
        // 32 sums in registers, keeps the shifts (the two extra live words per row cost it registers); with the sums
        // parked the permute measured 3-5% faster (17408 x 5120 T = 4 19.3 against 20.0 us).
        const uint32_t hb[2] = {((qh & 0xFu) * 0x204081u) & 0x01010101u, ((qh >> 4) * 0x204081u) & 0x01010101u};
#pragma unroll
        for (int k = 0; k < 8; k++)
          g[k] = lut[__builtin_amdgcn_perm(hb[k / 4], w[2 * r + k / 4], 0x0C0C0000u | ((4u + (k & 3)) << 8) | (k & 3))];
      } else {
#pragma unroll
        for (int k = 0; k < 8; k++) g[k] = lut[((w[2 * r + k / 4] >> (8 * (k & 3))) & 0xFF) | ((qh << (8 - k)) & 0x100)];
      }
#pragma unroll
      for (int p = 0; p < 4; p++) mm[p] = smask[(sg >> (8 * p)) & 0xFF];
      int sumi[NC];
#pragma unroll
      for (int c = 0; c < NC; c++) sumi[c] = 0;
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const uint32_t m = (k & 1) ? mm[k / 2].y : mm[k / 2].x;
        const int gs = (int)((g[k] ^ m) + (m & 0x01010101u));  // negated bytes: (b ^ 0xFF) + 1, no carry (b >= 1)
#pragma unroll
        for (int c = 0; c < NC; c++) sumi[c] = dot4(gs, u[c][k], sumi[c]);
      }
      const int mul = 1 + 2 * (int)((w[26] >> (4 * r)) & 0xF);
      const float d = (r & 1) ? half_hi(w[27 + r / 2]) : half_lo(w[27 + r / 2]);
#pragma unroll
      for (int c = 0; c < NC; c++) {
        const float t = (d * dy[c]) * (float)mul24(sumi[c], mul);
        acc_add<PARK, NC>(acc, park, r, c, t);
      }
    }
  } else if constexpr (TYPE == kIQ4XS) {
#pragma unroll
    for (int r = 0; r < 8; r++) {
      int sumi[NC];
#pragma unroll
      for (int c = 0; c < NC; c++) sumi[c] = 0;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint32_t q = w[4 * r + j];
        const int lo = iq4_levels(q & 0x0F0F0F0Fu, kv), hi = iq4_levels((q >> 4) & 0x0F0F0F0Fu, kv);
#pragma unroll
        for (int c = 0; c < NC; c++) sumi[c] = dot4(hi, u[c][j + 4], dot4(lo, u[c][j], sumi[c]));
      }
      const int ls = (int)(int8_t)((w[32 + r / 4] >> (8 * (r & 3))) & 0xFF);
      const float d = (r & 1) ? half_hi(w[34 + r / 2]) : half_lo(w[34 + r / 2]);
#pragma unroll
      for (int c = 0; c < NC; c++) acc_add<PARK, NC>(acc, park, r, c, (d * dy[c]) * (float)mul24(sumi[c], ls));
    }
  } else if constexpr (TYPE == kQ2K) {
    int s8a[NC], s8b[NC];  // activation sums of the two 16-weight halves (the min terms multiply them)
#pragma unroll
    for (int c = 0; c < NC; c++) {
      int ta = 0, tb = 0;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        ta = dot4(u[c][k], 0x01010101, ta);
        tb = dot4(u[c][k + 4], 0x01010101, tb);
      }
      s8a[c] = ta;
      s8b[c] = tb;
    }
#pragma unroll
    for (int r = 0; r < 8; r++) {
      int sa[NC], sb[NC];
#pragma unroll
      for (int c = 0; c < NC; c++) sa[c] = sb[c] = 0;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int va = (int)((w[2 * r] >> (2 * i)) & 0x03030303u), vb = (int)((w[2 * r + 1] >> (2 * i)) & 0x03030303u);
#pragma unroll
        for (int c = 0; c < NC; c++) {
          sa[c] = dot4(va, u[c][i], sa[c]);
          sb[c] = dot4(vb, u[c][4 + i], sb[c]);
        }
      }
      const uint32_t g = w[16 + r / 2] >> (16 * (r & 1));
      const int g0 = (int)(g & 0xFF), g1 = (int)((g >> 8) & 0xFF);
      const float d = half_lo(w[20 + r]), dmin = half_hi(w[20 + r]);
#pragma unroll
      for (int c = 0; c < NC; c++) {
        const int sd = mul24(sa[c], g0 & 0xF) + mul24(sb[c], g1 & 0xF);
        const int smn = mul24(s8a[c], g0 >> 4) + mul24(s8b[c], g1 >> 4);
        acc_add<PARK, NC>(acc, park, r, c, d * (dy[c] * (float)sd) - dmin * (dy[c] * (float)smn));
      }
    }
  } else if constexpr (TYPE == kIQ2XXS || TYPE == kIQ2XS || TYPE == kIQ2S) {
    // 64-bit codebook entries (8 magnitudes) in lut, then the byte masks of each sign byte (ksigns of 7 bits for
    // IQ2_XXS / IQ2_XS, the stored byte for IQ2_S)
    const uint2* grid = (const uint2*)lut;
    const uint2* smask = (const uint2*)(lut + LutInfo<TYPE>::grid);
#pragma unroll
    for (int r = 0; r < 8; r++) {
      uint2 e[4], mm[4];
#pragma unroll
      for (int p = 0; p < 4; p++) {
        if constexpr (TYPE == kIQ2XXS) {
          e[p] = grid[(w[2 * r] >> (8 * p)) & 0xFF];
          mm[p] = smask[(w[2 * r + 1] >> (7 * p)) & 0x7F];
        } else if constexpr (TYPE == kIQ2XS) {
          const uint32_t q16 = (w[2 * r + p / 2] >> (16 * (p & 1))) & 0xFFFF;
          e[p] = grid[q16 & 0x1FF];
          mm[p] = smask[q16 >> 9];
        } else {
          const uint32_t qh = (w[16 + r / 4] >> (8 * (r & 3))) & 0xFF;
          e[p] = grid[((w[r] >> (8 * p)) & 0xFF) | ((qh << (8 - 2 * p)) & 0x300)];
          mm[p] = smask[(w[8 + r] >> (8 * p)) & 0xFF];
        }
      }
      int s0[NC], s1[NC];
#pragma unroll
      for (int c = 0; c < NC; c++) s0[c] = s1[c] = 0;
#pragma unroll
      for (int p = 0; p < 4; p++) {
        const int gx = (int)((e[p].x ^ mm[p].x) + (mm[p].x & 0x01010101u));
        const int gy = (int)((e[p].y ^ mm[p].y) + (mm[p].y & 0x01010101u));
#pragma unroll
        for (int c = 0; c < NC; c++) {
          if (p < 2 || TYPE == kIQ2XXS) s0[c] = dot4(gy, u[c][2 * p + 1], dot4(gx, u[c][2 * p], s0[c]));
          else s1[c] = dot4(gy, u[c][2 * p + 1], dot4(gx, u[c][2 * p], s1[c]));
        }
      }
      if constexpr (TYPE == kIQ2XXS) {
        const int ls = (int)((w[2 * r + 1] >> 27) | 1);
        const float d = (r & 1) ? half_hi(w[16 + r / 2]) : half_lo(w[16 + r / 2]);
#pragma unroll
        for (int c = 0; c < NC; c++) acc_add<PARK, NC>(acc, park, r, c, (d * dy[c]) * (float)(mul24(s0[c], ls) / 8));
      } else {
        const uint32_t lsb = TYPE == kIQ2XS ? (w[16 + r / 4] >> (8 * (r & 3))) & 0xFF : (w[18 + r / 4] >> (8 * (r & 3))) & 0xFF;
        const int ls0 = (int)(lsb & 0xF), ls1 = (int)(lsb >> 4);
        constexpr int DW = TYPE == kIQ2XS ? 18 : 20;
        const float d = (r & 1) ? half_hi(w[DW + r / 2]) : half_lo(w[DW + r / 2]);
#pragma unroll
        for (int c = 0; c < NC; c++) {
          const int si = (mul24(s0[c], ls0) + mul24(s1[c], ls1) + (s0[c] + s1[c]) / 2) / 4;
          acc_add<PARK, NC>(acc, park, r, c, (d * dy[c]) * (float)si);
        }
      }
    }
  } else if constexpr (TYPE == kIQ3XXS) {
    const uint2* smask = (const uint2*)(lut + LutInfo<TYPE>::grid);
#pragma unroll
    for (int r = 0; r < 8; r++) {
      const uint32_t aux = w[16 + r];
      uint32_t g[8];
      uint2 mm[4];
#pragma unroll
      for (int k = 0; k < 8; k++) g[k] = lut[(w[2 * r + k / 4] >> (8 * (k & 3))) & 0xFF];
#pragma unroll
      for (int p = 0; p < 4; p++) mm[p] = smask[(aux >> (7 * p)) & 0x7F];
      int sumi[NC];
#pragma unroll
      for (int c = 0; c < NC; c++) sumi[c] = 0;
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const uint32_t m = (k & 1) ? mm[k / 2].y : mm[k / 2].x;
        const int gs = (int)((g[k] ^ m) + (m & 0x01010101u));
#pragma unroll
        for (int c = 0; c < NC; c++) sumi[c] = dot4(gs, u[c][k], sumi[c]);
      }
      const int ls = (int)(aux >> 28);
      const float d = (r & 1) ? half_hi(w[24 + r / 2]) : half_lo(w[24 + r / 2]);
#pragma unroll
      for (int c = 0; c < NC; c++) {
        const int si = (mul24(ls, sumi[c]) + sumi[c] / 2) / 2;
        acc_add<PARK, NC>(acc, park, r, c, (d * dy[c]) * (float)si);
      }
    }
  } else if constexpr (TYPE == kIQ1M) {
    int sy[NC][4];  // activation sums of the 4 groups of 8 (the delta term multiplies them)
#pragma unroll
    for (int c = 0; c < NC; c++)
#pragma unroll
      for (int p = 0; p < 4; p++) sy[c][p] = dot4(u[c][2 * p + 1], 0x01010101, dot4(u[c][2 * p], 0x01010101, 0));
#pragma unroll
    for (int r = 0; r < 8; r++) {
      const uint32_t qs = w[r];
      const uint32_t qh16 = (w[8 + r / 2] >> (16 * (r & 1))) & 0xFFFF;
      uint32_t grid[4];
#pragma unroll
      for (int p = 0; p < 4; p++) grid[p] = lut[((qs >> (8 * p)) & 0xFF) | ((((qh16 >> (4 * p)) & 7)) << 8)];
      int si[NC][2];
      float sf[NC][2];
#pragma unroll
      for (int c = 0; c < NC; c++) {
        si[c][0] = si[c][1] = 0;
        sf[c][0] = sf[c][1] = 0.0f;
      }
#pragma unroll
      for (int p = 0; p < 4; p++) {
        const int g0 = (int)(grid[p] & 0x0F0F0F0Fu), g1 = (int)((grid[p] >> 4) & 0x0F0F0F0Fu);
        const float delta = ((qh16 >> (4 * p)) & 8) ? -1.125f : -0.875f;
#pragma unroll
        for (int c = 0; c < NC; c++) {
          si[c][p / 2] = dot4(g1, u[c][2 * p + 1], dot4(g0, u[c][2 * p], si[c][p / 2]));
          sf[c][p / 2] += delta * (float)sy[c][p];
        }
      }
      const uint32_t sc6 = (w[12 + r / 4] >> (8 * (r & 3))) & 0xFF;
      const float sc0 = (float)(2 * (int)(sc6 & 7) + 1), sc1 = (float)(2 * (int)((sc6 >> 3) & 7) + 1);
      const float d = (r & 1) ? half_hi(w[14 + r / 2]) : half_lo(w[14 + r / 2]);
#pragma unroll
      for (int c = 0; c < NC; c++)
        acc_add<PARK, NC>(acc, park, r, c, (d * dy[c]) * ((((float)si[c][0] + sf[c][0]) * sc0) + (((float)si[c][1] + sf[c][1]) * sc1)));
    }
  }
}

// Value of lane (lane ^ O) over the whole wave.
template <int O>
__device__ __forceinline__ float xchg(float v) {
  if constexpr (O == 32) return lane_xor32(v);
  else return lane_xor<O>(v);
}
// One butterfly level over the first CUR live values: lanes with bit O set keep the upper half, the others the lower
// half; each adds the partner's copy of the same values. The two candidates are chosen with bit masks (v_bfi), so no
// value is ever selected by a per-lane index (which the compiler would lower to a compare chain over all values).
template <int O, int CUR, int V>
__device__ __forceinline__ void reduce_level(float (&a)[V], int lane) {
  if constexpr (CUR > 1) {
    constexpr int h = CUR / 2;
    const int up = (lane & O) ? -1 : 0;
#pragma unroll
    for (int i = 0; i < h; i++) {
      const int lo = __builtin_bit_cast(int, a[i]), hi = __builtin_bit_cast(int, a[i + h]);
      const float send = __builtin_bit_cast(float, (lo & up) | (hi & ~up));
      const float keep = __builtin_bit_cast(float, (hi & up) | (lo & ~up));
      a[i] = keep + xchg<O>(send);
    }
  } else {
    a[0] += xchg<O>(a[0]);
  }
}
// Waves per tile, a function of the type, K and the column count only (part of the summation order). One column, and
// two for all types but IQ3_XXS / IQ3_S / IQ1_M: one block of each tile per lane, ceil(K / 2048) waves, up to K = 32768
// (16 waves); each wave adds a butterfly, which is cheap for few columns. Otherwise, and for K > 32768: at most 4 waves,
// lanes taking several blocks. Measured (us, 5120 x 17408, 4 -> 9 waves): T = 1 Q4_K 13.1 -> 10.9, IQ3_S 18.0 -> 12.5,
// IQ2_XXS 14.7 -> 9.7; T = 2 Q4_K 14.7 -> 13.5, IQ2_S 19.3 -> 14.7, but IQ3_S 15.8 -> 20.1, IQ1_M 18.1 -> 21.5; T = 4
// Q4_K 18.7 -> 25.4.
constexpr int kMaxW = 16;
constexpr int waves_per_tile(int type, int K, int ncols) {
  const int w = (K / 256 + 7) / 8;
  const bool wide = ncols == 1 || (ncols == 2 && type != kIQ3XXS && type != kIQ3S && type != kIQ1M);
  const int cap = wide ? kMaxW : 4;
  return w < 1 ? 1 : w > kMaxW ? 4 : w > cap ? cap : w;
}

// FUSED: the activations arrive as f32 (xf, [NC][K]); every workgroup first quantizes them to q8_1 in LDS with the
// code of quantize_q8_1 (q8_1_store_n: amax, d = amax / 127, q = roundf(y / d), scale fp16(d)), then reads them from
// there. The results are those of quantize_q8_1 followed by the unfused GEMV, bit for bit.
constexpr int kFusedMaxX = 40960;  // NC * K values a fused launch may quantize per workgroup (40 KB of int8 in LDS)
template <int TYPE, int NC, bool NTP, bool ONE, bool FUSED = false>
__device__ __forceinline__ void qgemv_body(Mat m, const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                           float* __restrict__ y, int K, int W, const float* __restrict__ xf = nullptr) {
  constexpr int LW = LutInfo<TYPE>::words;
  __shared__ uint32_t lut[LW > 0 ? LW : 1];
  __shared__ float part[kMaxW][8 * NC];
  if constexpr (FUSED) {
    __shared__ __align__(16) int8_t s_xq[kFusedMaxX];
    __shared__ float s_xd[kFusedMaxX / 32];
    const int nblk = NC * K / 32;
    const int lane8 = threadIdx.x & 7;
    for (int b = threadIdx.x >> 3; b < nblk; b += blockDim.x >> 3) {
      const int i0 = 32 * b + block_offset(lane8);
      const float4 v = ld4(xf + i0);
      const float yv[1][4] = {{v.x, v.y, v.z, v.w}};
      q8_1_store_n<false, 1, true>(yv, s_xq, s_xd, nullptr, i0, 0);
    }
    xq = s_xq;
    xd = s_xd;
    __syncthreads();
  }
  if constexpr (LW > 0) {
    constexpr int G = LutInfo<TYPE>::grid, NM = LutInfo<TYPE>::masks;
    for (int i = threadIdx.x; i < G; i += blockDim.x) {
      uint32_t v;
      if constexpr (TYPE == kIQ3S) v = kIQ3SGrid[i];
      else if constexpr (TYPE == kIQ3XXS) v = kIQ3XXSGrid[i];
      else if constexpr (TYPE == kIQ1M) v = kIQ1SGrid[i];
      else if constexpr (TYPE == kIQ2XXS) v = (uint32_t)(kIQ2XXSGrid[i / 2] >> (32 * (i & 1)));
      else if constexpr (TYPE == kIQ2XS) v = (uint32_t)(kIQ2XSGrid[i / 2] >> (32 * (i & 1)));
      else v = (uint32_t)(kIQ2SGrid[i / 2] >> (32 * (i & 1)));
      lut[i] = v;
    }
    for (int i = threadIdx.x; i < NM; i += blockDim.x) {
      const int sb = NM == 128 ? (i | ((__builtin_popcount(i) & 1) << 7)) : i;  // ksigns: even count of negatives
      uint32_t m0 = 0, m1 = 0;
      for (int j = 0; j < 4; j++) {
        m0 |= ((sb >> j) & 1) ? 0xFFu << (8 * j) : 0u;
        m1 |= ((sb >> (4 + j)) & 1) ? 0xFFu << (8 * j) : 0u;
      }
      lut[G + 2 * i] = m0;
      lut[G + 2 * i + 1] = m1;
    }
  }
  uint32_t kv[4] = {0, 0, 0, 0};
  if constexpr (TYPE == kIQ4XS) {
#pragma unroll
    for (int i = 0; i < 4; i++)
      kv[i] = (uint32_t)(uint8_t)kIQ4NL[4 * i] | ((uint32_t)(uint8_t)kIQ4NL[4 * i + 1] << 8) |
              ((uint32_t)(uint8_t)kIQ4NL[4 * i + 2] << 16) | ((uint32_t)(uint8_t)kIQ4NL[4 * i + 3] << 24);
  }
  if constexpr (LW > 0) __syncthreads();
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int tile = blockIdx.x;
  const int wv = wave;
  const int lb = lane >> 3, s = lane & 7;
  const bool live = tile < m.ntiles;  // uniform per wave
  float acc[8 * NC];
#pragma unroll
  for (int i = 0; i < 8 * NC; i++) acc[i] = 0.0f;
  if (live) {
    // Blocks b, b + step, ... of this lane, software-pipelined: the next chunk is requested right after the current
    // block's activations (so waiting for those does not wait for the prefetch; loads return in order) and before
    // the current chunk is decoded. Past the last block the prefetch re-reads the current block (a cache hit), so
    // every load is unconditional.
    const int step = 8 * W;
    int b = 8 * wv + lb;
    Chunk<TYPE> ca, cb;
    int u[NC][8];
    float dy[NC];
    auto load_x = [&](int bb) {
#pragma unroll
      for (int c = 0; c < NC; c++) {
        const int4* xp = (const int4*)(xq + (size_t)c * K + (size_t)bb * 256 + s * 32);
        const int4 a0 = xp[0], a1 = xp[1];
        u[c][0] = a0.x; u[c][1] = a0.y; u[c][2] = a0.z; u[c][3] = a0.w;
        u[c][4] = a1.x; u[c][5] = a1.y; u[c][6] = a1.z; u[c][7] = a1.w;
        dy[c] = xd[(size_t)c * (K / 32) + bb * 8 + s];
      }
    };
    if constexpr (ONE && !FUSED && NC == 4 && parks_sums(TYPE)) {
      // four columns: the 16 sums of rows 0-3 parked in LDS row by row keep the chunk's decode in fewer VGPRs (IQ3_S:
      // 90 instead of a 128-VGPR cap and a 12-byte spill to scratch); the values and their order are unchanged
      __shared__ float park[4 * NC][256];
      if (b < m.nb) {
        load_chunk<TYPE, NTP>(ca, m, (size_t)tile, b, s);
        load_x(b);
        dot_chunk<TYPE, NC, true>(ca, u, dy, lut, kv, acc, &park[0][threadIdx.x]);
        asm volatile("" ::: "memory");  // the sums come back from LDS, not from registers the compiler kept
#pragma unroll
        for (int i = 0; i < 4 * NC; i++) acc[i] = park[i][threadIdx.x];
      }
    } else if constexpr (ONE) {
      if (b < m.nb) {
        load_chunk<TYPE, NTP>(ca, m, (size_t)tile, b, s);
        load_x(b);
        dot_chunk<TYPE, NC>(ca, u, dy, lut, kv, acc);
      }
    } else {
      if (b < m.nb) load_chunk<TYPE, NTP>(ca, m, (size_t)tile, b, s);
      while (b < m.nb) {
        load_x(b);
        const int b1 = b + step;
        load_chunk<TYPE, NTP>(cb, m, (size_t)tile, b1 < m.nb ? b1 : b, s);
        dot_chunk<TYPE, NC>(ca, u, dy, lut, kv, acc);
        if (b1 >= m.nb) break;
        load_x(b1);
        const int b2 = b1 + step;
        load_chunk<TYPE, NTP>(ca, m, (size_t)tile, b2 < m.nb ? b2 : b1, s);
        dot_chunk<TYPE, NC>(cb, u, dy, lut, kv, acc);
        b = b2;
      }
    }
  }
  // 64-lane butterfly; afterwards lane l holds value index l >> (6 - log2(8 NC)) (copies in the lower lane bits)
  constexpr int V = 8 * NC;
  constexpr int c1 = V, c2 = c1 > 1 ? c1 / 2 : 1, c3 = c2 > 1 ? c2 / 2 : 1, c4 = c3 > 1 ? c3 / 2 : 1,
                c5 = c4 > 1 ? c4 / 2 : 1, c6 = c5 > 1 ? c5 / 2 : 1;
  reduce_level<32, c1>(acc, lane);
  reduce_level<16, c2>(acc, lane);
  reduce_level<8, c3>(acc, lane);
  reduce_level<4, c4>(acc, lane);
  reduce_level<2, c5>(acc, lane);
  reduce_level<1, c6>(acc, lane);
  constexpr int shift = V == 8 ? 3 : V == 16 ? 2 : V == 32 ? 1 : 0;  // NC = 3 (V = 24) is handled on the host
  const int idx = lane >> shift;
  const bool writer = (lane & ((1 << shift) - 1)) == 0;
  if (W == 1) {
    if (live && writer) y[(size_t)(idx % NC) * m.N + tile * 8 + idx / NC] = acc[0];
    return;
  }
  if (writer) part[wave][idx] = acc[0];
  __syncthreads();
  if (live && wv == 0 && writer) {
    float t = part[wave][idx];
    for (int k = 1; k < W; k++) t = t + part[wave + k][idx];
    y[(size_t)(idx % NC) * m.N + tile * 8 + idx / NC] = t;
  }
}

// Kernel for K <= 2048 W (every lane takes at most one block of its tile): no prefetch registers, and the compiler is
// held to 128 VGPRs (4 waves per SIMD) for four columns. Measured against the prefetching kernel (us, 17408 x 5120,
// T = 1 / T = 4): Q4_K 10.9 -> 9.8 / 17.3 -> 17.9, Q6_K 14.7 -> 13.1 / 20.0 -> 19.3, IQ3_S 13.2 -> 11.4 / 20.3 -> 19.3,
// IQ2_S 15.9 -> 12.1 / 24.4 -> 23.4, IQ4_XS 11.7 -> 11.1 / 18.3 -> 17.4, Q2_K 9.3 -> 7.8 / 17.2 -> 18.8 (Q2_K and
// Q4_K with four columns keep the prefetching kernel). The additions are the same, so the results are identical.
// Its wide pieces are always read with nontemporal loads: ordinary loads at K = 17408 measured 2-5% slower (Q6_K T = 1
// 13.7 -> 14.3 us), the opposite of the prefetching kernel.
// IQ3_S with four columns needed a few more than 128 VGPRs here and spilled 12 bytes per lane to scratch (about 2 MB
// of scratch traffic per 17408 x 5120 launch) until the sums of half the rows were parked in LDS (parks_sums).
#ifndef Q27H_QG_WPE_ONE
#define Q27H_QG_WPE_ONE 4
#endif
template <int TYPE, int NC, bool NTP, bool FUSED = false>
__global__ void __launch_bounds__(256) qgemv_kernel(Mat m, const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                    float* __restrict__ y, int K, int W, const float* __restrict__ xf) {
  qgemv_body<TYPE, NC, NTP, false, FUSED>(m, xq, xd, y, K, W, xf);
}
template <int TYPE, int NC, bool FUSED = false>
__global__ void __launch_bounds__(64 * kMaxW) __attribute__((amdgpu_waves_per_eu(Q27H_QG_WPE_ONE)))
qgemv_one_kernel(Mat m, const int8_t* __restrict__ xq, const float* __restrict__ xd, float* __restrict__ y, int K, int W,
                 const float* __restrict__ xf) {
  qgemv_body<TYPE, NC, true, true, FUSED>(m, xq, xd, y, K, W, xf);
}

int check_type(int type) {
  if (fmt_of(type).nf == 0) return fail(Q27H_ERR_UNSUPPORTED, "qgemv: weight type " + std::to_string(type) + " not supported");
  return Q27H_OK;
}

template <int TYPE, int NC, bool FUSED = false>
void launch_gemv(const Mat& m, const int8_t* xq, const float* xd, float* y, int K, hipStream_t s, const float* xf = nullptr) {
  const int W = waves_per_tile(TYPE, K, NC);
  const int grid = m.ntiles;
  // the prefetching kernel takes at most 4 waves (lanes with several blocks); W > 4 means one block per lane
  const bool one = m.nb <= 8 * W && (W > 4 || !((TYPE == kQ2K || TYPE == kQ4K) && NC == 4));
  if (one)
    hipLaunchKernelGGL((qgemv_one_kernel<TYPE, NC, FUSED>), dim3(grid), dim3(64 * W), 0, s, m, xq, xd, y, K, W, xf);
  else if (K <= kNtPiecesMaxK)
    hipLaunchKernelGGL((qgemv_kernel<TYPE, NC, true, FUSED>), dim3(grid), dim3(64 * W), 0, s, m, xq, xd, y, K, W, xf);
  else
    hipLaunchKernelGGL((qgemv_kernel<TYPE, NC, false, FUSED>), dim3(grid), dim3(64 * W), 0, s, m, xq, xd, y, K, W, xf);
}

template <int TYPE, bool FUSED = false>
void launch_nc(const Mat& m, const int8_t* xq, const float* xd, float* y, int K, int nc, hipStream_t s,
               const float* xf = nullptr) {
  if (nc == 1) launch_gemv<TYPE, 1, FUSED>(m, xq, xd, y, K, s, xf);
  else if (nc == 2) launch_gemv<TYPE, 2, FUSED>(m, xq, xd, y, K, s, xf);
  else launch_gemv<TYPE, 4, FUSED>(m, xq, xd, y, K, s, xf);
}

}  // namespace
}  // namespace q27h

using namespace q27h;

extern "C" size_t q27h_qmat_bytes(int type, int N, int K) {
  if (fmt_of(type).nf == 0 || N <= 0 || K <= 0 || N % 8 || K % 256) return 0;
  size_t off[5];
  return layout(type, N, K, off);
}

extern "C" int q27h_qgemv_waves(int type, int K, int ncols) {
  return waves_per_tile(type, K, ncols);
}

extern "C" int q27h_qmat_repack(int type, int N, int K, const void* raw, void* buf, q27h_stream_t s) {
  if (int e = check_type(type)) return e;
  if (N <= 0 || K <= 0 || N % 8 || K % 256) return fail(Q27H_ERR_SHAPE, "qmat_repack: N % 8 and K % 256 must be 0");
  if (!raw || !buf) return fail(Q27H_ERR_ARG, "qmat_repack: null pointer");
  if (((uintptr_t)buf & 255u) != 0) return fail(Q27H_ERR_ARG, "qmat_repack: buf needs 256-byte alignment");
  size_t off[5];
  layout(type, N, K, off);
  uint8_t* b = (uint8_t*)buf;
  const int nb = K / 256;
  const dim3 grid((unsigned)((size_t)(N / 8) * ((nb + kRepackBlocks - 1) / kRepackBlocks)));
  const uint8_t* r = (const uint8_t*)raw;
#define Q27H_REPACK(T) hipLaunchKernelGGL(repack_kernel<T>, grid, dim3(256), 0, stream_of(s), r, b + off[0], b + off[1], b + off[2], \
                                           b + off[3], b + off[4], nb)
  switch (type) {
    case kQ2K: Q27H_REPACK(kQ2K); break;
    case kQ4K: Q27H_REPACK(kQ4K); break;
    case kQ6K: Q27H_REPACK(kQ6K); break;
    case kIQ2XXS: Q27H_REPACK(kIQ2XXS); break;
    case kIQ2XS: Q27H_REPACK(kIQ2XS); break;
    case kIQ3XXS: Q27H_REPACK(kIQ3XXS); break;
    case kIQ3S: Q27H_REPACK(kIQ3S); break;
    case kIQ2S: Q27H_REPACK(kIQ2S); break;
    case kIQ1M: Q27H_REPACK(kIQ1M); break;
    default: Q27H_REPACK(kIQ4XS); break;
  }
#undef Q27H_REPACK
  return check_launch("qmat_repack");
}

extern "C" int q27h_qgemv(int type, int N, int K, const void* buf, const int8_t* xq, const float* xd, float* y, int ncols,
                          q27h_stream_t s) {
  if (int e = check_type(type)) return e;
  if (N <= 0 || K <= 0 || N % 8 || K % 256) return fail(Q27H_ERR_SHAPE, "qgemv: N % 8 and K % 256 must be 0");
  if (ncols < 1 || ncols > 4) return fail(Q27H_ERR_SHAPE, "qgemv: ncols must be 1..4");
  if (!buf || !xq || !xd || !y) return fail(Q27H_ERR_ARG, "qgemv: null pointer");
  if (((uintptr_t)buf & 255u) != 0 || !aligned16(xq)) return fail(Q27H_ERR_ARG, "qgemv: buf needs 256-byte and xq 16-byte alignment");
  size_t off[5];
  layout(type, N, K, off);
  const uint8_t* b = (const uint8_t*)buf;
  const Mat m{{b + off[0], b + off[1], b + off[2], b + off[3]}, b + off[4], N, K / 256, N / 8};
  const hipStream_t st = stream_of(s);
  // three columns run as two launches (columns 0-1, then column 2), each with its own rows of y
  auto run = [&](const int8_t* q, const float* d, float* yy, int nc) {
    switch (type) {
      case kQ2K: launch_nc<kQ2K>(m, q, d, yy, K, nc, st); break;
      case kQ4K: launch_nc<kQ4K>(m, q, d, yy, K, nc, st); break;
      case kQ6K: launch_nc<kQ6K>(m, q, d, yy, K, nc, st); break;
      case kIQ2XXS: launch_nc<kIQ2XXS>(m, q, d, yy, K, nc, st); break;
      case kIQ2XS: launch_nc<kIQ2XS>(m, q, d, yy, K, nc, st); break;
      case kIQ3XXS: launch_nc<kIQ3XXS>(m, q, d, yy, K, nc, st); break;
      case kIQ3S: launch_nc<kIQ3S>(m, q, d, yy, K, nc, st); break;
      case kIQ2S: launch_nc<kIQ2S>(m, q, d, yy, K, nc, st); break;
      case kIQ1M: launch_nc<kIQ1M>(m, q, d, yy, K, nc, st); break;
      default: launch_nc<kIQ4XS>(m, q, d, yy, K, nc, st); break;
    }
  };
  if (ncols == 3) {
    run(xq, xd, y, 2);
    run(xq + (size_t)2 * K, xd + (size_t)2 * (K / 32), y + (size_t)2 * N, 1);
  } else {
    run(xq, xd, y, ncols);
  }
  return check_launch("qgemv");
}

extern "C" int q27h_qgemv_f32(int type, int N, int K, const void* buf, const float* x, float* y, int ncols,
                              q27h_stream_t s) {
  if (int e = check_type(type)) return e;
  if (N <= 0 || K <= 0 || N % 8 || K % 256) return fail(Q27H_ERR_SHAPE, "qgemv_f32: N % 8 and K % 256 must be 0");
  if (ncols < 1 || ncols > 4) return fail(Q27H_ERR_SHAPE, "qgemv_f32: ncols must be 1..4");
  if ((long)K * (ncols == 3 ? 2 : ncols) > kFusedMaxX)
    return fail(Q27H_ERR_SHAPE, "qgemv_f32: K * ncols must be at most " + std::to_string(kFusedMaxX) + " (q8_1 activations in LDS)");
  if (!buf || !x || !y) return fail(Q27H_ERR_ARG, "qgemv_f32: null pointer");
  if (((uintptr_t)buf & 255u) != 0 || !aligned16(x)) return fail(Q27H_ERR_ARG, "qgemv_f32: buf needs 256-byte and x 16-byte alignment");
  size_t off[5];
  layout(type, N, K, off);
  const uint8_t* b = (const uint8_t*)buf;
  const Mat m{{b + off[0], b + off[1], b + off[2], b + off[3]}, b + off[4], N, K / 256, N / 8};
  const hipStream_t st = stream_of(s);
  auto run = [&](const float* xx, float* yy, int nc) {
    switch (type) {
      case kQ2K: launch_nc<kQ2K, true>(m, nullptr, nullptr, yy, K, nc, st, xx); break;
      case kQ4K: launch_nc<kQ4K, true>(m, nullptr, nullptr, yy, K, nc, st, xx); break;
      case kQ6K: launch_nc<kQ6K, true>(m, nullptr, nullptr, yy, K, nc, st, xx); break;
      case kIQ2XXS: launch_nc<kIQ2XXS, true>(m, nullptr, nullptr, yy, K, nc, st, xx); break;
      case kIQ2XS: launch_nc<kIQ2XS, true>(m, nullptr, nullptr, yy, K, nc, st, xx); break;
      case kIQ3XXS: launch_nc<kIQ3XXS, true>(m, nullptr, nullptr, yy, K, nc, st, xx); break;
      case kIQ3S: launch_nc<kIQ3S, true>(m, nullptr, nullptr, yy, K, nc, st, xx); break;
      case kIQ2S: launch_nc<kIQ2S, true>(m, nullptr, nullptr, yy, K, nc, st, xx); break;
      case kIQ1M: launch_nc<kIQ1M, true>(m, nullptr, nullptr, yy, K, nc, st, xx); break;
      default: launch_nc<kIQ4XS, true>(m, nullptr, nullptr, yy, K, nc, st, xx); break;
    }
  };
  if (ncols == 3) {
    run(x, y, 2);
    run(x + (size_t)2 * K, y + (size_t)2 * N, 1);
  } else {
    run(x, y, ncols);
  }
  return check_launch("qgemv_f32");
}
