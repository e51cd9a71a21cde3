/* CPU oracle for the fused per-layer ops: TEST INFRASTRUCTURE ONLY.
 *
 * A scalar C restatement of the reference engine's fused ops (src/ops.cu, src/prefill.cu, src/qgemv.cu,
 * src/common.cuh, src/requant.cpp of avallavall/qwen27-engine), used by tests/ and by bench.py's
 * cpu_baseline leg as the checker. The product library never links, loads or calls it.
 *
 * Every function reproduces the float-operation order of the reference kernel it names, with these
 * contract decisions (the reference itself is built with -use_fast_math, whose values no CPU can
 * reproduce):
 *   - no FP contraction anywhere (compile with -ffp-contract=off);
 *   - rsqrtf(x) is 1.0f / sqrtf(x), both correctly rounded;
 *   - expf / logf are q27o_expf / q27o_logf (Cody-Waite reduction + polynomial, defined below), sin/cos of
 *     RoPE angles are q27o_sincos (Cody-Waite reduction in double + Taylor polynomials, rounded to float);
 *   - the RoPE frequency of pair j is powf(theta_scale, (float)j) evaluated once on the host;
 *   - reductions follow the reference's 32-lane xor butterflies over its thread layout exactly.
 * Parity status of each function is listed in the header of q27_oracle.c.
 */
#ifndef Q27_ORACLE_H
#define Q27_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar math shared by every op */
float q27o_expf(float x);
float q27o_logf(float x);
void q27o_sincos(float theta, float* s, float* c);
float q27o_silu(float x);
float q27o_sigmoid(float x);
float q27o_softplus(float x);
uint16_t q27o_f2h(float f);
float q27o_h2f(uint16_t h);
uint16_t q27o_f2bf(float f);
float q27o_bf2f(uint16_t b);
void q27o_rope_freqs(float theta_scale, float* freq32);

/* ---- q8_1 / element-wise / norms (decode and prefill) */
void q27o_quantize_q8_1(const float* x, int8_t* xq, float* xd, int K, int ncols, float* xs);
void q27o_rmsnorm(const float* x, const float* w, float* y, int n, int rows, float eps, int ystride);
void q27o_add(const float* x, const float* a, float* y, int n);
void q27o_swiglu(const float* g, const float* u, float* y, int n);
void q27o_rmsnorm_q8(const float* x, const float* w, float* h, int8_t* xq, float* xd, int n, int rows, float eps, float* xs);
void q27o_sum_norm_q8(float* x, const float* partial, int n, int rows, const float* w, float eps, float* h, int8_t* xq,
                      float* xd);
void q27o_sum_norm_rows(float* x, const float* partial, int n, int M, const float* w, float eps, float* h, int8_t* xq,
                        float* xd, float* xs);
void q27o_add_norm_rows(float* x, const float* partial, const uint16_t* recv_bf16, int n, int M, const float* w, float eps,
                        float* h, int8_t* xq, float* xd, float* xs);
/* gemv_bf16_pair (src/ops.cu:377-393) */
void q27o_gemv_bf16_pair(const uint16_t* Wa, const uint16_t* Wb, const float* x, float* ya, float* yb, int N, int K, int T);
/* wire formats of the two-card sum (src/prefill.cu:338-406); qb = values per fp16 scale (16 or 32) */
void q27o_to_bf16(const float* x, uint16_t* y, size_t n);
void q27o_to_q8_wire(const float* partial, float* ef, int first, uint8_t* wire, int n, int M, int qb);
void q27o_add_norm_rows_q8(float* x, const uint8_t* own, const uint8_t* recv, int n, int M, const float* w, float eps,
                           float* h, int8_t* xq, float* xd, float* xs, int qb);
void q27o_swiglu_q8(const float* g, const float* u, int8_t* xq, float* xd, int n, float* xs);
void q27o_gated_rmsnorm(const float* o, const float* w, const float* z, float* y, int n, int heads, float eps);
void q27o_gated_rmsnorm_q8(const float* o, const float* w, const float* z, int8_t* xq, float* xd, int heads, float eps,
                           float* xs);
void q27o_l2norm_heads(float* x, int n, int heads, int T, int stride, float eps);

/* ---- Gated-DeltaNet input stage */
void q27o_gdn_gates(const float* a, const float* b, const float* ssm_a, const float* dt_bias, float* g, float* beta, int H,
                    int T);
void q27o_gdn_conv(const float* x, const float* w, float* planes, int in_plane, float* y, int C, int T, int snapshots);
void q27o_gdn_conv_l2(const float* x, const float* w, float* planes, int in_plane, float* y, int C, int T, int snapshots,
                      int n_norm_heads, float eps, const float* a, const float* b, const float* ssm_a, const float* dt_bias,
                      float* g, float* beta, int H);
void q27o_gdn_conv_prefill(const float* x, const float* w, float* planes, int in_plane, float* y, int C, int M,
                           int n_norm_heads, float eps, const float* a, const float* b, const float* ssm_a,
                           const float* dt_bias, float* g, float* beta, int H);
/* gdn_step (q27_oracle_gdn.c): the delta-rule recurrence of src/ops.h:40-45. */
int q27o_gdn_step(const float* q, const float* k, const float* v, int stride, const float* g, const float* beta,
                  float* planes, int in_plane, float* o, int H, int HK, int T, float scale, int snapshots, int flip);
/* the same with the part count (8 or 16) as an argument */
int q27o_gdn_step_parts(int parts, const float* q, const float* k, const float* v, int stride, const float* g,
                        const float* beta, float* planes, int in_plane, float* o, int H, int HK, int T, float scale,
                        int snapshots, int flip);

/* ---- attention input stage: Q/K RMSNorm + (IM)RoPE + KV-cache write */
size_t q27o_kv_cache_bytes(int nkvh, int n_ctx, int q8);
void q27o_attn_prep(const float* qg, const float* k, const float* v, const float* q_norm, const float* k_norm, float* qn,
                    void* kcache, void* vcache, int pos0, int T, float eps, float theta_scale, int nqh, int nkvh, int n_ctx,
                    int q8, const int* rope3, const int* rdelta);

/* ---- quantized embedding gather (GGUF blocks) */
void q27o_get_rows_iq2_s(const uint8_t* table, int64_t row_bytes, const int* ids, int T, float* y, int n, const float* img);
void q27o_get_rows_q4_k(const uint8_t* table, int64_t row_bytes, const int* ids, int T, float* y, int n, const float* img);
void q27o_get_rows_q6_k(const uint8_t* table, int64_t row_bytes, const int* ids, int T, float* y, int n, const float* img);
void q27o_get_rows_q8_0(const uint8_t* table, int64_t row_bytes, const int* ids, int T, float* y, int n, const float* img);
const uint64_t* q27o_iq2s_grid(void);

/* ---- decode GEMV over quantized weights (q27_oracle_qgemv.c): raw GGUF rows, q8_1 activations, ncols 1..4.
 * Types: ggml ids 12 (Q4_K), 14 (Q6_K), 21 (IQ3_S), 23 (IQ4_XS). Returns 0, or -1 for a bad shape / type. */
int q27o_qgemv_block_bytes(int type);
int q27o_qgemv_waves(int type, int K, int ncols);
int q27o_qgemv(int type, const uint8_t* raw, int N, int K, const int8_t* xq, const float* xd, float* y, int ncols);

#ifdef __cplusplus
}
#endif
#endif
