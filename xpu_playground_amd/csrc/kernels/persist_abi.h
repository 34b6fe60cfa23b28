// Argument blocks of the persistent Qwen3 decode kernel
// (kernels/qwen3_persist.hip), shared by the kernel and the engine
// (qwen3_engine.cpp), which fills them in device memory.
#pragma once

#include <stdint.h>

struct xpu_persist_layer {
  const uint16_t *qkv, *o, *gu, *down, *in_norm, *post_norm, *q_norm, *k_norm;
  uint16_t *kc, *vc;  // this layer's chunk-major K and V caches
};

struct xpu_persist_args {
  const struct xpu_persist_layer *layers;
  const uint16_t *embed, *final_norm, *lm_head, *cos_t, *sin_t;
  uint16_t *x, *qkv, *attn, *h, *logits;
  float *part_val;
  uint32_t *part_idx, *part_bad;
  uint32_t *state;  // [0] position, [1] input token, [2] last argmax, [3] prompt length
  const uint32_t *prompt;
  uint32_t *gen;
  uint32_t *flags;  // 6 stage arrays of one word per block
  uint32_t *error;  // nonzero: a wait gave up (or the host stopped the grid); every block stops
  uint32_t layers_n, hidden, inter, vocab, heads, kv_heads, max_seq, gen_capacity;
  float eps, scale;
  uint32_t spin_limit;  // polls before a wait gives up
  uint32_t pad;
};
