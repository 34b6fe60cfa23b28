/*
 * CPU oracle for the xpu_playground decode hot path (GEMV, GEMM, Qwen3 decode).
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product library links, loads or
 * calls this code; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, and only as the checker / CPU baseline.
 *
 * Every function cites the reference file:line whose behaviour it restates
 * (paths relative to the xpu_playground repository root). Where the
 * reference's arithmetic lives in third-party code (qwen3/reference.py calls
 * transformers==4.51.0 Qwen3ForCausalLM in eager bf16, qwen3/requirements.txt:2),
 * the restated rounding points are those of modeling_qwen3.py: RMSNorm
 * bf16(w * bf16(x * rsqrt(mean(x^2) + eps))), linear = bf16(fp32 dot),
 * RoPE bf16(bf16(q*cos) + bf16(rotate_half(q)*sin)), eager attention
 * bf16 scores * scale -> bf16, fp32 softmax -> bf16 probabilities,
 * bf16(P.V), SiLU bf16(silu(g)) then bf16(* up), residual bf16(a + b).
 *
 * Summation orders. The reference fixes no FP32 summation order for the
 * decode (transformers calls oneDNN). The oracle therefore fixes one
 * ("canonical order", below) and the gfx950 kernels implement the same one,
 * so the GPU decode can be compared bit for bit. The reference's own order
 * (gemv.cpp:126-134: one sequential FP32 sum per row) is restated separately
 * (orc_gemv_rows_seq) for its known-answer check, and an FP64 reference
 * (orc_gemv_f64, orc_gemm_f64) bounds both.
 *
 * Canonical order of a length-n FP32 sum of terms t_k (orc_canonical_*):
 *   element k goes to lane L = (k / 8) % 64, slot e = k % 8, chunk j = k / 512;
 *   acc[L][e] starts at +0.0f and, for j ascending, acc[L][e] += t_k
 *   (a fused multiply-add when t_k is a product; products of two bf16 or two
 *   fp16 values are exact in FP32, so fma and mul+add agree);
 *   lane sum s[L] = ((acc0+acc1)+(acc2+acc3)) + ((acc4+acc5)+(acc6+acc7));
 *   then for m = 32,16,8,4,2,1: s[L] = s[L] + s[L ^ m]; result s[0].
 * Sums longer than 4096 terms that the attention kernel splits (the softmax
 * denominator) are taken per 4096-term chunk and the chunk sums are added
 * in ascending chunk order starting from +0.0f.
 */
#ifndef XPU_ORACLE_H
#define XPU_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- codecs: qwen3/model.cpp:497-508, level_zero/peak_l0.cpp:726-785 ---- */
uint16_t orc_f32_to_bf16(float v);
float orc_bf16_to_f32(uint16_t v);
uint16_t orc_f32_to_fp16(float v);
float orc_fp16_to_f32(uint16_t v);
/* dtype: 0 = bf16, 1 = fp16 */
uint16_t orc_encode(float v, int dtype);
float orc_decode(uint16_t v, int dtype);
void orc_encode_n(const float *in, uint16_t *out, size_t n, int dtype);
void orc_decode_n(const uint16_t *in, float *out, size_t n, int dtype);

/* ---- seeded synthetic inputs ---- */
uint64_t orc_hash(uint64_t seed, uint64_t index);
/* U[-1,1) 24-bit uniforms rounded to dtype codes */
void orc_fill_uniform(uint16_t *out, uint64_t n, uint64_t seed, int dtype);
/* N(0, std^2) via Box-Muller in double, rounded to float then bf16 codes */
void orc_fill_normal_bf16(uint16_t *out, uint64_t n, uint64_t seed, float stddev);
/* bf16 codes of 1 + N(0, std^2) (norm gains for tests); std=0 gives 1.0 */
void orc_fill_gain_bf16(uint16_t *out, uint64_t n, uint64_t seed, float stddev);
/* uniform token ids in [0, vocab) */
void orc_fill_tokens(uint32_t *out, uint64_t n, uint64_t seed, uint32_t vocab);
/* gemv.cpp:91-103 hash initialisation (matrix in [0.25,0.5), vector in [0.5,0.75)) */
void orc_fill_reference_gemv(uint16_t *matrix, uint16_t *vector, uint32_t m,
                             uint32_t k, uint32_t ld, int dtype);

/* ---- GEMV ---- */
/* gemv.cpp:126-134 / peak_l0.cpp:866-885: y_r = sequential FP32 sum over k */
void orc_gemv_rows_seq(const uint16_t *a, const uint16_t *x, float *y,
                       uint32_t rows, uint32_t k, uint64_t lda, int dtype);
/* FP64 accumulation, all rows (multithreaded) */
void orc_gemv_f64(const uint16_t *a, const uint16_t *x, double *y, uint32_t m,
                  uint32_t k, uint64_t lda, int dtype);
/* canonical order, rounded to dtype codes: the value the gfx950 GEMV returns */
void orc_gemv_canonical(const uint16_t *a, const uint16_t *x, uint16_t *y,
                        uint32_t m, uint32_t k, uint64_t lda, int dtype);
float orc_canonical_dot(const uint16_t *a, const uint16_t *x, uint32_t k, int dtype);
float orc_canonical_sum(const float *t, uint32_t n);
/* reference-order FP32 GEMV timed as the CPU baseline; returns seconds */
double orc_time_gemv_seq(const uint16_t *a, const uint16_t *x, float *y,
                         uint32_t m, uint32_t k, int dtype, int threads);

/* ---- GEMM (gemm.cpp:73-117, peak_l0.cpp:895-949) ---- */
void orc_gemm_f64(const uint16_t *a, const uint16_t *b, double *c, uint32_t m,
                  uint32_t n, uint32_t k, int dtype, const uint32_t *rows,
                  uint32_t nrows);
/* FP32 ascending-k accumulation of selected rows (reference check order) */
void orc_gemm_f32_rows(const uint16_t *a, const uint16_t *b, float *c, uint32_t m,
                       uint32_t n, uint32_t k, int dtype, const uint32_t *rows,
                       uint32_t nrows);
/* same sums as orc_gemm_f32_rows (all m rows), cache-blocked; bitwise equal */
void orc_gemm_f32_blocked(const uint16_t *a, const uint16_t *b, float *c, uint32_t m,
                          uint32_t n, uint32_t k, int dtype);
/* wall seconds of orc_gemm_f32_blocked on `threads` threads */
double orc_time_gemm_blocked(const uint16_t *a, const uint16_t *b, float *c, uint32_t m,
                             uint32_t n, uint32_t k, int dtype, int threads);
double orc_time_gemm_f32(const uint16_t *a, const uint16_t *b, float *c,
                         uint32_t m, uint32_t n, uint32_t k, int dtype,
                         uint32_t row_limit, int threads);

/* ---- Qwen3 primitives (qwen3/kernels.hpp:24-246 with transformers rounding) ---- */
typedef struct {
  uint32_t hidden, intermediate, layers, heads, kv_heads, head_dim, vocab;
  float rms_eps;
  double rope_theta;
  uint32_t tied; /* lm_head == embed_tokens */
} orc_qwen3_config;

float orc_exp(float x);
void orc_rmsnorm(const uint16_t *x, const uint16_t *w, uint16_t *out,
                 uint32_t width, float eps);
void orc_rope_tables(uint16_t *cos_t, uint16_t *sin_t, uint32_t max_seq,
                     uint32_t head_dim, double theta);
/* q/k: bf16 head vectors (modified in place like QkvRopeCache) */
void orc_qk_norm_rope(uint16_t *vec, const uint16_t *norm_w, const uint16_t *cos_row,
                      const uint16_t *sin_row, uint32_t head_dim, float eps);
/* attention of one query head over cache rows 0..n-1 (row t at kcache + t*stride) */
void orc_attention_head(const uint16_t *q, const uint16_t *kcache,
                        const uint16_t *vcache, uint64_t stride, uint32_t n,
                        uint32_t head_dim, uint16_t *out);
void orc_add(uint16_t *left, const uint16_t *right, uint32_t width);
void orc_silu_mul(uint16_t *gate, const uint16_t *up, uint32_t width);
uint32_t orc_argmax(const uint16_t *logits, uint32_t width);

/* ---- Qwen3 engine (qwen3/main.cpp:118-329) ---- */
typedef struct orc_qwen3 orc_qwen3;
/* weight kinds for orc_qwen3_tensor */
enum {
  ORC_W_Q = 0, ORC_W_K = 1, ORC_W_V = 2, ORC_W_O = 3, ORC_W_QNORM = 4,
  ORC_W_KNORM = 5, ORC_W_GATE = 6, ORC_W_UP = 7, ORC_W_DOWN = 8,
  ORC_W_INNORM = 9, ORC_W_POSTNORM = 10, ORC_W_EMBED = 11, ORC_W_FINALNORM = 12,
  ORC_W_LMHEAD = 13
};
uint64_t orc_qwen3_tensor_elems(const orc_qwen3_config *c, int kind);
void orc_qwen3_fill_tensor(const orc_qwen3_config *c, uint64_t seed, float gain_std,
                           int kind, uint32_t layer, uint16_t *out);
orc_qwen3 *orc_qwen3_create(const orc_qwen3_config *c, uint64_t seed,
                            float gain_std, uint32_t max_seq);
void orc_qwen3_destroy(orc_qwen3 *m);
uint16_t *orc_qwen3_weight(orc_qwen3 *m, int kind, uint32_t layer);
/* one decode step; returns the argmax token (0xffffffff on NaN/Inf); logits
 * (bf16 codes, vocab entries) copied out when logits != NULL */
uint32_t orc_qwen3_decode(orc_qwen3 *m, uint32_t token, uint32_t position,
                          uint16_t *logits);
/* hidden state x after the last decode step (bf16 codes, hidden entries) */
const uint16_t *orc_qwen3_hidden(orc_qwen3 *m);
/* prompt + greedy loop (main.cpp:342-352); returns number generated */
uint32_t orc_qwen3_generate(orc_qwen3 *m, const uint32_t *prompt, uint32_t n_prompt,
                            uint32_t max_new, uint32_t stop_on_eos, uint32_t *out,
                            uint16_t *logits_steps, uint32_t n_logit_steps);
void orc_set_threads(int n);
int orc_get_threads(void);

#ifdef __cplusplus
}
#endif
#endif
