/*
 * xpu_qwen3.h - batch-1 greedy Qwen3 decode on gfx950 (C ABI).
 *
 * Replaces the reference engine qwen3/main.cpp:118-329 (Engine: weight
 * arena, KV caches, RoPE tables, decode(token, position)) and its command
 * line (main.cpp:17-102,333-363), shape-parameterised (the reference accepts
 * only Qwen3-8B, qwen3/model.cpp:395-408) and with tied embeddings.
 *
 * Numerics follow transformers' eager bf16 Qwen3 (the arithmetic of the
 * reference oracle qwen3/reference.py): every linear layer is a bf16 GEMV
 * with FP32 accumulation, activations are bf16, RMSNorm / QK-norm / RoPE /
 * attention / SiLU round where transformers rounds.
 *
 * Modes: XPU_QWEN3_GRAPH (default) runs the fused kernels of one token as a
 * captured HIP graph (decode position and token live in device memory);
 * XPU_QWEN3_EAGER launches the same fused kernels one by one;
 * XPU_QWEN3_REFERENCE runs the reference's eight kernel entries with
 * blocking launches in the reference's order (main.cpp:159-226). All modes
 * produce identical bits.
 */
#ifndef XPU_QWEN3_H
#define XPU_QWEN3_H

#include "xpu_runtime.h"

#ifdef __cplusplus
extern "C" {
#endif

/* qwen3/model.hpp:11-22 and config.json fields (model.cpp:376-393);
 * head_dim must be 128, heads a multiple of kv_heads; tied = 1 means
 * lm_head.weight is model.embed_tokens.weight. */
typedef struct {
  uint32_t hidden, intermediate, layers, heads, kv_heads, head_dim, vocab;
  float rms_eps;
  double rope_theta;
  uint32_t tied;
} xpu_qwen3_config;

#define XPU_QWEN3_GRAPH 0
#define XPU_QWEN3_EAGER 1
#define XPU_QWEN3_REFERENCE 2

/* Tensor kinds for the synthetic generator (one seed stream each);
 * XPU_W_LMHEAD only exists for untied configs. */
#define XPU_W_Q 0
#define XPU_W_K 1
#define XPU_W_V 2
#define XPU_W_O 3
#define XPU_W_QNORM 4
#define XPU_W_KNORM 5
#define XPU_W_GATE 6
#define XPU_W_UP 7
#define XPU_W_DOWN 8
#define XPU_W_INNORM 9
#define XPU_W_POSTNORM 10
#define XPU_W_EMBED 11
#define XPU_W_FINALNORM 12
#define XPU_W_LMHEAD 13

typedef struct xpu_qwen3 xpu_qwen3;

/* Presets: "qwen3-0.6b" (BASELINE workload), "qwen3-8b" (the reference's
 * shape, untied), "tiny", "small" (test shapes). */
int xpu_qwen3_preset(const char *name, xpu_qwen3_config *out);

/* Host-side synthetic weights: matrices N(0, 0.02^2) and norm gains
 * 1 + N(0, gain_std^2) (exactly 1 for gain_std = 0), bf16 codes, generated
 * by Box-Muller from the counter hash of (seed, kind, layer, index).
 * count must equal the tensor's element count. */
int xpu_qwen3_fill_tensor(const xpu_qwen3_config *cfg, uint64_t seed, float gain_std, int kind,
                          uint32_t layer, uint16_t *out, uint64_t count);

/* RoPE tables [max_seq][head_dim] in bf16 (replaces Engine::upload_rope,
 * main.cpp:299-318, with transformers' FP32 angle). */
int xpu_qwen3_rope_tables(uint16_t *cos_t, uint16_t *sin_t, uint32_t max_seq, uint32_t head_dim,
                          double theta);

/* Seeded token ids uniform in [0, vocab). */
int xpu_synth_tokens(uint32_t *out, uint64_t n, uint64_t seed, uint32_t vocab);

/* Create an engine on rt (NULL: the engine creates and owns a runtime on
 * the default device) with synthetic weights (seed, gain_std), KV caches
 * for max_seq positions (<= 40960, main.cpp:69-70). */
int xpu_qwen3_create(xpu_runtime *rt, const xpu_qwen3_config *cfg, uint32_t max_seq, uint64_t seed,
                     float gain_std, xpu_qwen3 **out);
/* Read and validate <model_dir>/config.json (host only; model.cpp:376-410
 * generalised to the Qwen3 family: model_type qwen3, hidden_act silu,
 * dtype bfloat16, no rope_scaling, head_dim 128). */
int xpu_qwen3_read_config(const char *model_dir, xpu_qwen3_config *out);

/* Host-only check of a checkpoint directory, the counterpart of
 * load_and_validate_checkpoint (qwen3/model.cpp:448-495): the config as
 * xpu_qwen3_read_config; with model.safetensors.index.json, every
 * weight_map shard's header lists exactly the tensors mapped to it and
 * metadata.total_size equals the payload bytes; every tensor is BF16 and
 * lies inside its shard's payload, no two payloads of a shard overlap; the
 * tensor set and shapes are those of the config. XPU_ERR_INVALID with the
 * reason otherwise. out (may be NULL) receives the config. */
int xpu_qwen3_validate_checkpoint(const char *model_dir, xpu_qwen3_config *out);

/* Same, loading a Hugging Face checkpoint directory (config.json,
 * model.safetensors[.index.json]) with bf16 tensors (model.cpp:448-495). */
int xpu_qwen3_create_from_checkpoint(xpu_runtime *rt, const char *model_dir, uint32_t max_seq,
                                     xpu_qwen3 **out);
void xpu_qwen3_destroy(xpu_qwen3 *eng);
int xpu_qwen3_get_config(const xpu_qwen3 *eng, xpu_qwen3_config *out);

/* Select the mode for the following calls. Reference mode keeps the KV
 * caches position-major ([layer][position][kv_head][128], as
 * qwen3/main.cpp:131-137), graph and eager modes chunk-major, in the same
 * buffers; graph and eager modes may alternate within a sequence. A decode
 * at position > 0 whose mode's layout differs from the one the sequence was
 * started in fails with XPU_ERR_INVALID: after switching between reference
 * and graph/eager mode, start again at position 0 (generate always does). */
int xpu_qwen3_set_mode(xpu_qwen3 *eng, int mode);

/* Prompt processing in xpu_qwen3_generate (graph and eager modes), mode:
 *   0 stepwise: the prompt goes through decode one position at a time, as
 *     the reference does (main.cpp:343-344);
 *   1 batched (default when the module has kernels for the shape): the
 *     prompt positions run as one batch per layer with the same arithmetic
 *     as the decode step (the last position's last-layer MLP, final norm,
 *     lm_head and argmax on the decode step's own kernels), so the KV
 *     caches, tokens and logits are bit-identical to stepwise;
 *   2 gemm: as batched in chunks of up to 4096 positions, with the four
 *     projections on the MFMA GEMM and the causal attention on MFMA (FP32
 *     sums in the MFMA's order, the hardware exp), so the caches differ
 *     from stepwise by rounding, not bitwise.
 * XPU_ERR_INVALID for another mode or a mode without kernels for the
 * shape. The reference has no batched prompt path. */
int xpu_qwen3_set_prefill(xpu_qwen3 *eng, int mode);

/* Attention of the graph and eager modes for contexts of at least
 * min_context positions (position + 1 >= min_context) runs split over
 * compute units: a scores kernel over 256-position tiles and a P.V kernel
 * per 16 output dims, with the same operations in the same order as the
 * one-block-per-head kernel, so results are bit-identical; each variant has
 * its own captured graph. 0 never splits. Default 257. No reference counterpart:
 * the reference's Attention (qwen3/kernels.hpp:157-192) is one serial loop
 * per head. XPU_ERR_INVALID when the module lacks the kernels. */
int xpu_qwen3_set_attention_split(xpu_qwen3 *eng, uint32_t min_context);

/* One forward step at `position` for input `token`; *next = greedy token
 * (Engine::decode, main.cpp:159-226). A non-finite logit fails with
 * XPU_ERR_VERIFY ("model produced a NaN or infinity", main.cpp:223-224). */
int xpu_qwen3_decode(xpu_qwen3 *eng, uint32_t token, uint32_t position, uint32_t *next);

/* bf16 logits (vocab entries) / hidden state (hidden entries) of the last step */
int xpu_qwen3_logits(xpu_qwen3 *eng, uint16_t *out, uint64_t count);
int xpu_qwen3_hidden(xpu_qwen3 *eng, uint16_t *out, uint64_t count);

/* Prompt + greedy loop (main.cpp:342-352): the prompt goes through decode one
 * position at a time (or the batched forms, xpu_qwen3_set_prefill); token i
 * of out is the argmax after position n_prompt - 1 + i; stops after an EOS id (151645, 151643) when
 * stop_on_eos. *n_out = number of ids written. prompt_ms / decode_ms (may be
 * NULL): device time of the prompt steps and of the n_out - 1 decode steps. */
int xpu_qwen3_generate(xpu_qwen3 *eng, const uint32_t *prompt, uint32_t n_prompt, uint32_t max_new,
                       int stop_on_eos, uint32_t *out, uint32_t *n_out, double *prompt_ms,
                       double *decode_ms);

/* Command line with the reference's flags (main.cpp:17-72):
 *   --model-dir DIR | --synthetic PRESET [--seed N] [--gain-std X]
 *   --input-ids FILE|- --max-new-tokens N [--max-seq-len N]
 *   [--mode graph|eager|reference] [--prefill batched|gemm|stepwise] [--no-eos-stop]
 * prints {"generated_ids":[...]} on stdout, diagnostics on stderr. */
int run_qwen3(int argc, char **argv);

#ifdef __cplusplus
}
#endif
#endif
