/* q27h: C ABI of the MI355X (gfx950) fused per-layer ops of the qwen27 engine.
 *
 * Every entry point mirrors one launcher of the reference engine (avallavall/qwen27-engine) with the same
 * argument order and meaning, plain device pointers and an opaque stream (`q27h_stream_t` is a hipStream_t;
 * NULL = the default stream). Each call only enqueues work on that stream and returns; nothing synchronises
 * the host, and device-resident scalars (positions, plane index, ids) are read on the device, so every call
 * may be recorded in a HIP graph. Return value: Q27H_OK, or a negative code with q27h_last_error() holding
 * the message (per host thread). The C++ header q27/ops.h re-exposes the reference's exact signatures on
 * top of these and throws std::runtime_error on a non-zero status.
 *
 * Layout rules shared by all entry points: rows are contiguous ([rows][n]); float arrays read or written four
 * values at a time must be 16-byte aligned (any row offset of a 5120-wide or 128-wide array keeps this);
 * q8_1 outputs are xq int8 [..][K], xd f32 [..][K/32] (the value of the fp16-rounded scale) and the optional
 * xs f32 [..][K/16] (sums of the unquantized values per 16).
 */
#ifndef Q27H_H
#define Q27H_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define Q27H_ABI_VERSION 1

#define Q27H_OK 0
#define Q27H_ERR_SHAPE (-1)       /* a size the reference launcher rejects (std::runtime_error there) */
#define Q27H_ERR_UNSUPPORTED (-2) /* a feature outside this build: the two-GPU exchange arguments */
#define Q27H_ERR_HIP (-3)         /* a HIP runtime error at launch */
#define Q27H_ERR_ARG (-4)         /* null or misaligned pointer */
#define Q27H_ERR_FORMAT (-5)      /* a malformed or unsupported GGUF file (std::runtime_error in the reference) */
#define Q27H_ERR_IO (-6)          /* a file that cannot be opened or mapped */
#define Q27H_ERR_NOT_FOUND (-7)   /* a missing GGUF key or tensor */

typedef void* q27h_stream_t;

const char* q27h_last_error(void);
int q27h_abi_version(void);

/* ---------------------------------------------------------------- element-wise and unfused norms */
/* rmsnorm (src/ops.h:15, src/ops.cu:746-748): y = x * rsqrt(mean(x^2) + eps) * w per row; ystride 0 = n. */
int q27h_rmsnorm(const float* x, const float* w, float* y, int n, int rows, float eps, q27h_stream_t s, int ystride);
/* add (src/ops.h:17, src/ops.cu:749-751): y = x + a over n values. */
int q27h_add(const float* x, const float* a, float* y, int n, q27h_stream_t s);
/* swiglu (src/ops.h:19, src/ops.cu:752-754): y = silu(g) * u over n values. */
int q27h_swiglu(const float* g, const float* u, float* y, int n, q27h_stream_t s);
/* set_int (src/ops.h:45, src/ops.cu:744): *p = v, enqueued. */
int q27h_set_int(int* p, int v, q27h_stream_t s);

/* ---------------------------------------------------------------- q8_1 producers (fused) */
/* rmsnorm_q8 (src/ops.h:99-100, src/ops.cu:697-701): RMSNorm of `rows` rows of n = 5120 -> h (may be NULL),
 * q8_1 xq/xd and xs (may be NULL). */
int q27h_rmsnorm_q8(const float* x, const float* w, float* h, int8_t* xq, float* xd, int n, int rows, float eps,
                    q27h_stream_t s, float* xs);
/* sum_norm_q8 (src/ops.h:103-104, src/ops.cu:702-722): x += partial in place, then rmsnorm_q8 of x (no xs).
 * `ar` is the reference's two-card ArArgs: must be NULL here (Q27H_ERR_UNSUPPORTED otherwise). pf/pf_bytes
 * (an L2 prefetch hint of the next GEMV's weights) are accepted and ignored. n must be 5120. */
int q27h_sum_norm_q8(float* x, const float* partial, int n, int rows, const void* ar, const float* w, float eps, float* h,
                     int8_t* xq, float* xd, q27h_stream_t s, const void* pf, size_t pf_bytes);
/* sum_norm_rows (src/prefill.h:31-32, src/prefill.cu:489-501): prefill form of sum_norm_q8 with xs; `ex` (the
 * reference's PfExchange) must be NULL. */
int q27h_sum_norm_rows(float* x, const float* partial, int n, int M, const void* ex, const float* w, float eps, float* h,
                       int8_t* xq, float* xd, float* xs, q27h_stream_t s);
/* add_norm_rows (src/prefill.h:46-47, src/prefill.cu:516-520): x += partial (recv NULL) or
 * x += bf16(partial) + recv (recv = bf16 bits [M][n]), then RMSNorm -> h (may be NULL), q8_1 and xs. */
int q27h_add_norm_rows(float* x, const float* partial, const uint16_t* recv, int n, int M, const float* w, float eps,
                       float* h, int8_t* xq, float* xd, float* xs, q27h_stream_t s);
/* quantize_q8_1 (src/qmat.h:50, src/qgemv.cu:840-845): x[ncols][K] -> q8_1 (+ xs). K % 32 == 0. */
int q27h_quantize_q8_1(const float* x, int8_t* xq, float* xd, int K, int ncols, q27h_stream_t s, float* xs);
/* swiglu_q8 (src/ops.h:106, src/ops.cu:723-726): silu(g) * u -> q8_1 (+ xs) over n values, n % 32 == 0. */
int q27h_swiglu_q8(const float* g, const float* u, int8_t* xq, float* xd, int n, q27h_stream_t s, float* xs);
/* gated_rmsnorm_q8 (src/ops.h:108-109, src/ops.cu:727-730): per head of 128,
 * (rms_norm(o) * w) * silu(z) -> q8_1 (+ xs), `heads` heads (tokens x value heads). */
int q27h_gated_rmsnorm_q8(const float* o, const float* w, const float* z, int8_t* xq, float* xd, int heads, float eps,
                          q27h_stream_t s, float* xs);
/* gated_rmsnorm (src/ops.h:43, src/ops.cu:794-796): the unfused form, y = (rms_norm_n(o) * w) * silu(z). */
int q27h_gated_rmsnorm(const float* o, const float* w, const float* z, float* y, int n, int heads, float eps,
                       q27h_stream_t s);

/* ---------------------------------------------------------------- Gated-DeltaNet input stage */
/* l2norm_heads (src/ops.h:34, src/ops.cu:781-783): x <- rms_norm(x, eps/n) / sqrt(n) per head of n values;
 * `heads` heads at the start of each of T rows of `stride` values. In place. */
int q27h_l2norm_heads(float* x, int n, int heads, int T, int stride, float eps, q27h_stream_t s);
/* gemv_bf16_pair (src/ops.h:24-26, src/ops.cu:377-393, 768-771): ya[t] = Wa x[t], yb[t] = Wb x[t] for two bf16
 * matrices of N rows and K columns (ssm_alpha / ssm_beta), f32 x [T][K], in the reference's summation order.
 * K % 8 == 0; Wa, Wb, x 16-byte aligned. */
int q27h_gemv_bf16_pair(const uint16_t* Wa, const uint16_t* Wb, const float* x, float* ya, float* yb, int N, int K, int T,
                        q27h_stream_t s);
/* gdn_gates (src/ops.h:29-30, src/ops.cu:773-776): beta = sigmoid(b), g = softplus(a + dt_bias) * ssm_a, [T][H]. */
int q27h_gdn_gates(const float* a, const float* b, const float* ssm_a, const float* dt_bias, float* g, float* beta, int H,
                   int T, q27h_stream_t s);
/* gdn_conv (src/ops.h:32-33, src/ops.cu:777-780): 4-tap causal conv + SiLU over C channels and T <= 4 tokens;
 * planes [4][C][3]; *in_plane (device) selects the input state. */
int q27h_gdn_conv(const float* x, const float* w, float* planes, const int* in_plane, float* y, int C, int T, int snapshots,
                  q27h_stream_t s);
/* gdn_step (src/ops.h:40-45, src/ops.cu:449-572 and 784-793): the gated delta rule over T tokens for H value heads
 * of 128 x 128 f32 state (value head h uses key head h % HK); q / k / v rows of `stride` floats (q, k at
 * kh * 128, v at h * 128), g / beta [T][H], o [T][H][128] = (S^T q) * scale. planes [4][H][128 col][128 i].
 * flip = 0 (decode, T <= 4): read plane *in_plane, write plane t after token t when snapshots, else plane T - 1.
 * flip = 1 (prefill, any T): the final state goes to plane (*in_plane == 0 ? 1 : 0); no snapshots. From T >= 128 on
 * this runs q27h_gdn_step_chunked (below) unless q27h_gdn_prefill_exact(1) was called or o overlaps an input: o and the
 * final state then agree with the sequential kernel within float32 rounding (relative 1e-5 per 128-value vector), not
 * bit for bit, and T is limited to 65535 * 32. Below 128 tokens, in exact mode or with an overlapping o, the
 * sequential kernel runs and its results are bit-exact against the CPU checker.
 * q, k and planes 16-byte aligned, stride % 4 == 0. */
int q27h_gdn_step(const float* q, const float* k, const float* v, int stride, const float* g, const float* beta,
                  float* planes, const int* in_plane, float* o, int H, int HK, int T, float scale, int snapshots,
                  q27h_stream_t s, int flip);
/* gdn_step's prefill (flip) mode in the chunked form on matrix cores: no counterpart in the reference, whose
 * prefill kernel runs token by token (src/ops.cu:449-572). Same arguments, outputs and plane semantics as
 * q27h_gdn_step with flip = 1 and snapshots = 0; the additions happen in another order, so o and the final state
 * agree with the sequential form to float32 rounding (relative 1e-5 per 128-value vector: a (token, head) row of o,
 * a state column), not bit for bit. q27h_gdn_step with flip = 1 takes this path for T >= 128 unless
 * q27h_gdn_prefill_exact(1) was called. o may share no byte with the q / k / v rows, g, beta or the planes (the
 * chunks' matrices are staged in o before the outputs overwrite them): Q27H_ERR_ARG otherwise. T <= 65535 * 32. */
int q27h_gdn_step_chunked(const float* q, const float* k, const float* v, int stride, const float* g,
                          const float* beta, float* planes, const int* in_plane, float* o, int H, int HK, int T,
                          float scale, q27h_stream_t s);
/* Process-wide choice for the Gated-DeltaNet prefill path: 1 = the CPU checker's bits (gdn_step's prefill (flip)
 * mode always on the sequential kernel, gdn_conv_prefill's SiLU correctly rounded), 0 (the default) = the faster
 * forms within the fp32 tolerance of 1e-5 relative (the chunked recurrence from 128 tokens on, the hardware
 * exp2 / reciprocal SiLU and rsq L2 scale in gdn_conv_prefill). Returns the previous setting. No counterpart
 * in the reference (its prefill is sequential); for callers that need the sequential bits. The setting is read when
 * q27h_gdn_step enqueues its launch: a graph captured under one setting keeps that path at every replay, and a thread
 * that changes it races with other threads' calls (a caller that needs a fixed path can call
 * q27h_gdn_step_chunked directly, or set exact mode once at start-up). */
int q27h_gdn_prefill_exact(int on);
/* gdn_conv_l2 (src/ops.h:112-114, src/ops.cu:731-737): gdn_conv + l2norm_heads of the first n_norm_heads heads
 * + gdn_gates in one launch. C % 128 == 0 and C / 128 - n_norm_heads == H. pf/pf_bytes ignored. */
int q27h_gdn_conv_l2(const float* x, const float* w, float* planes, const int* in_plane, float* y, int C, int T,
                     int snapshots, int n_norm_heads, float eps, const float* a, const float* b, const float* ssm_a,
                     const float* dt_bias, float* g, float* beta, int H, q27h_stream_t s, const void* pf, size_t pf_bytes);
/* gdn_conv_prefill (src/prefill.h:14-16, src/prefill.cu:479-485): the same over M tokens; the conv state after
 * the batch goes to plane (*in_plane == 0 ? 1 : 0). y's SiLU and the q / k heads' L2 scale are evaluated on the
 * hardware exp2, reciprocal and reciprocal square root (relative error below 4.1e-6 where |y| is normal, under the
 * 1e-5 fp32 bar), not bit for bit, unless q27h_gdn_prefill_exact(1) was called; the state planes, g and beta are
 * bit-exact either way. */
int q27h_gdn_conv_prefill(const float* x, const float* w, float* planes, const int* in_plane, float* y, int C, int M,
                          int n_norm_heads, float eps, const float* a, const float* b, const float* ssm_a,
                          const float* dt_bias, float* g, float* beta, int H, q27h_stream_t s);
/* gdn_flip_plane (src/prefill.h:18, src/prefill.cu:487): *plane = (*plane == 0 ? 1 : 0), enqueued. */
int q27h_gdn_flip_plane(int* plane, q27h_stream_t s);
/* flip_plane_to (src/prefill.h:41, src/prefill.cu:515): *dst = (*src == 0 ? 1 : 0), enqueued. */
int q27h_flip_plane_to(int* dst, const int* src, q27h_stream_t s);
/* The wire formats of the two-card partial sum (src/prefill.h:34-44, src/prefill.cu:338-370,503-513); the transfer
 * between cards is not part of this library. A q8 wire row of n = 5120 values is n int8 values, then n / qb fp16
 * scales (qb = 16 "q8b16", 32 "q8"; the reference picks it from Q27_WIRE, src/ops.cu:20-30), 16-byte aligned.
 * to_bf16: y = bf16(x) (round to nearest even), n even.
 * to_q8_wire: per qb-value block of y = partial (+ ef unless first; ef may be NULL): q = roundf(y / (amax / 127)),
 *   scale fp16(amax / 127); ef <- y - scale * q (error feedback).
 * add_norm_rows_q8: x += (dequant(own) + dequant(recv)), then RMSNorm * w -> h (may be NULL), q8_1 and xs (may be
 *   NULL), as add_norm_rows. */
int q27h_to_bf16(const float* x, uint16_t* y, size_t n, q27h_stream_t s);
int q27h_to_q8_wire(const float* partial, float* ef, int first, uint8_t* wire, int n, int M, int qb, q27h_stream_t s);
int q27h_add_norm_rows_q8(float* x, const uint8_t* own, const uint8_t* recv, int n, int M, const float* w, float eps,
                          float* h, int8_t* xq, float* xd, float* xs, int qb, q27h_stream_t s);

/* ---------------------------------------------------------------- attention input stage */
/* kv_cache_bytes (src/ops.h:54, src/attn.cu:890-892): bytes of one layer's K (or V) cache:
 * q8 ? nkvh * n_ctx * (256 + 16) : nkvh * n_ctx * 512. */
size_t q27h_kv_cache_bytes(int nkvh, int n_ctx, int q8);
/* attn_prep (src/ops.h:59-62, src/ops.cu:798-803): per-head RMSNorm of q (nqh heads at stride 512 of qg) and k
 * (nkvh heads), NeoX RoPE of dims (j, j + 32), j < 32, with theta = p * theta_scale^j, p = rope3[t][j % 3]
 * (IMRoPE, rope3 [T][3] device, may be NULL) or *pos0 + t - *rdelta (rdelta may be NULL); qn [T][nqh][256];
 * K and V to cache row *pos0 + t: f16 [nkvh][n_ctx][256] (q8 = 0) or q8_0 int8 [nkvh][n_ctx][256] followed by
 * fp16 scales [nkvh][n_ctx][8]. Rows outside [0, n_ctx) are not written. pf/pf_bytes ignored. */
int q27h_attn_prep(const float* qg, const float* k, const float* v, const float* q_norm, const float* k_norm, float* qn,
                   void* kcache, void* vcache, const int* pos0, int T, float eps, float theta_scale, int nqh, int nkvh,
                   int n_ctx, int q8, q27h_stream_t s, const void* pf, size_t pf_bytes, const int* rope3,
                   const int* rdelta);

/* ---------------------------------------------------------------- quantized embedding gather */
/* get_rows_iq2_s (src/ops.h:22-23, src/ops.cu:756-766): rows ids[t] (device) of an IQ2_S table (82-byte
 * super-blocks, row_bytes apart) -> f32 y [T][n], n % 256 == 0; id < 0 copies row (-id - 1) of img [..][n]
 * (zeros when img is NULL). */
int q27h_get_rows_iq2_s(const uint8_t* table, int64_t row_bytes, const int* ids, int T, float* y, int n, q27h_stream_t s,
                        const float* img);
/* No reference kernel (the reference's embedding is IQ2_S only, src/model.cu:104-105); same signature and
 * id rule as get_rows_iq2_s, ggml block formats: Q4_K (144-byte super-blocks, ggml dequantize_row_q4_K as
 * transcribed in src/requant.cpp:90-114), Q6_K (210 bytes, src/requant.cpp:68-88), Q8_0 (34-byte blocks of
 * 32, y = q * fp16 d; n % 32 == 0). */
int q27h_get_rows_q4_k(const uint8_t* table, int64_t row_bytes, const int* ids, int T, float* y, int n, q27h_stream_t s,
                       const float* img);
int q27h_get_rows_q6_k(const uint8_t* table, int64_t row_bytes, const int* ids, int T, float* y, int n, q27h_stream_t s,
                       const float* img);
int q27h_get_rows_q8_0(const uint8_t* table, int64_t row_bytes, const int* ids, int T, float* y, int n, q27h_stream_t s,
                       const float* img);

/* ---------------------------------------------------------------- decode GEMV over quantized weights
 * Weight types are the ggml type ids of the reference's GEMV (src/gguf.h:12-14, src/qgemv.cu:63-71): 10 Q2_K, 12 Q4_K,
 * 14 Q6_K, 16 IQ2_XXS, 17 IQ2_XS, 18 IQ3_XXS, 21 IQ3_S, 22 IQ2_S, 23 IQ4_XS, 29 IQ1_M. A matrix of N rows
 * (outputs, N % 8 == 0) and K columns (K % 256 == 0) lives in one caller-owned device buffer in the tile layout
 * of the reference's QMat (src/qmat.h:1-8).
 * q27h_qmat_bytes (src/qmat.h:31): bytes of that buffer (0 for an unsupported type or shape). */
size_t q27h_qmat_bytes(int type, int N, int K);
/* Repack (the device half of qmat_upload, src/qmat.h:34, src/qgemv.cu:227-260): raw = N GGUF rows already in device
 * memory ([N][K/256] blocks), buf = q27h_qmat_bytes() bytes, 256-byte aligned. Byte moves only. */
int q27h_qmat_repack(int type, int N, int K, const void* raw, void* buf, q27h_stream_t s);
/* qgemv (src/qmat.h:44-46, src/qgemv.cu:785-801): y[c][n] = sum_k W[n][k] x[c][k] for c < ncols (1..4; the reference
 * takes 1, 2 or 4), x as q8_1 activations xq [ncols][K] (16-byte aligned), xd [ncols][K/32]. */
int q27h_qgemv(int type, int N, int K, const void* buf, const int8_t* xq, const float* xd, float* y, int ncols,
               q27h_stream_t s);
/* qgemv over f32 activations x [ncols][K] (16-byte aligned): no counterpart in the reference, which runs
 * quantize_q8_1 (src/qgemv.cu:840-845) and then qgemv (src/qgemv.cu:785-801) as two launches (src/model.cu:727-728,
 * 826-827). Every workgroup quantizes x to q8_1 in LDS with the code of q27h_quantize_q8_1, so y equals that pair's
 * result bit for bit; one launch instead of two, for callers whose activations are f32. K * ncols <= 40960
 * (K * 2 for three columns), else Q27H_ERR_SHAPE. Slower than the pair at the decode shapes (every workgroup
 * quantizes the whole x): 5120 x 6144 at four columns 21-23 against 12-13 us. */
int q27h_qgemv_f32(int type, int N, int K, const void* buf, const float* x, float* y, int ncols, q27h_stream_t s);
/* Waves that share one 8-row tile in a q27h_qgemv launch of ncols columns (1..16; three columns run as launches of two
 * and one): part of the summation order, a function of the type, K and ncols only. */
int q27h_qgemv_waves(int type, int K, int ncols);

/* ---------------------------------------------------------------- GGUF reader (src/gguf.h, src/gguf.cpp)
 * Version-3 files only, memory-mapped read-only for the life of the handle; tensor data pointers point into the
 * mapping (host memory). Errors: Q27H_ERR_IO (cannot open / map), Q27H_ERR_FORMAT with the reference's messages
 * ("not a GGUF file: ...", "GGUF version N not supported", "gguf: truncated file", "bad n_dims for ...",
 * "unknown ggml type N", "tensor out of file: ..."), Q27H_ERR_NOT_FOUND for a missing key or tensor. */
typedef struct q27h_gguf q27h_gguf;
/* GValue::Kind (src/gguf.h:33-41) */
#define Q27H_GV_INT 0
#define Q27H_GV_FLOAT 1
#define Q27H_GV_BOOL 2
#define Q27H_GV_STRING 3
#define Q27H_GV_ARR_INT 4
#define Q27H_GV_ARR_FLOAT 5
#define Q27H_GV_ARR_STRING 6
/* GTensor (src/gguf.h:21-30); name is NUL-terminated and owned by the handle. */
typedef struct {
  const char* name;
  size_t name_len;
  int type;
  int n_dims;
  int64_t ne[4];
  uint64_t offset;
  uint64_t nbytes;
  const uint8_t* data;
} q27h_gtensor;
/* GValue (src/gguf.h:33-41): scalars in i / f / s; arrays of n elements in ai / af (owned by the handle) or, for
 * strings, through q27h_gguf_kv_str_at. */
typedef struct {
  int kind;
  int64_t i;
  double f;
  const char* s;
  size_t s_len;
  uint64_t n;
  const int64_t* ai;
  const double* af;
} q27h_gvalue;
/* gtype_block_bytes / gtype_block_size / gtype_name (src/gguf.h:15-19, src/gguf.cpp:18-62); 0 / "?" for a type
 * the engine does not know (the reference throws). */
int q27h_gtype_block_bytes(int type);
int q27h_gtype_block_size(int type);
const char* q27h_gtype_name(int type);
/* GGUF::GGUF(path) / ~GGUF (src/gguf.h:46-47, src/gguf.cpp:113-194) */
int q27h_gguf_open(const char* path, q27h_gguf** out);
void q27h_gguf_close(q27h_gguf* g);
/* GGUF::tensors() / find() / tensor() (src/gguf.h:52-54): the index of `name` or -1; entry i (file order). */
int64_t q27h_gguf_n_tensors(const q27h_gguf* g);
int64_t q27h_gguf_find(const q27h_gguf* g, const char* name);
int q27h_gguf_tensor(const q27h_gguf* g, int64_t i, q27h_gtensor* out);
/* GGUF::has() / kv() (src/gguf.h:56-57). Keys are listed by index in file order; a key is returned as pointer +
 * length (it may hold any byte, NUL included, as the reference's std::string keys may), and q27h_gguf_kv_at /
 * q27h_gguf_kv_str_at address a key by that index. q27h_gguf_kv looks a NUL-terminated key up by name. */
int64_t q27h_gguf_n_kv(const q27h_gguf* g);
int q27h_gguf_key(const q27h_gguf* g, int64_t i, const char** s, size_t* len);
int q27h_gguf_kv(const q27h_gguf* g, const char* key, q27h_gvalue* out);
int q27h_gguf_kv_at(const q27h_gguf* g, int64_t i, q27h_gvalue* out);
int q27h_gguf_kv_str_at(const q27h_gguf* g, int64_t i, uint64_t j, const char** s, size_t* len);

/* Staged host -> device copy, the transfer of qmat_upload (src/qmat.h:34, which issues one cudaMemcpyAsync from
 * the pageable mapping): `bytes` from host `src` (e.g. a tensor's data in the mapping) to device `dst` on stream s,
 * in 16 MiB chunks that `threads` host threads (<= 0: up to 8) copy into six pinned staging buffers while the
 * previous chunks' DMA runs. Returns once the last DMA is enqueued; src may be reused at once. One call at a time per
 * process (internally serialised). */
int q27h_copy_h2d_staged(void* dst, const void* src, size_t bytes, int threads, q27h_stream_t s);
/* The same transfer for rows [row0, row0 + nrows) of tensor `tensor` of an open file, read with pread from the
 * file into the staging buffers (no page faults on the mapping): the upload path of qmat_upload when the caller
 * holds the GGUF. Q27H_ERR_SHAPE for rows outside the tensor, Q27H_ERR_IO if the file cannot be read. */
int q27h_gguf_upload_rows(const q27h_gguf* g, int64_t tensor, int64_t row0, int64_t nrows, void* dst, int threads,
                          q27h_stream_t s);

#ifdef __cplusplus
}
#endif
#endif
