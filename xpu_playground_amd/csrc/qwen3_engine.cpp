// Qwen3 batch-1 greedy decode engine on gfx950 (include/xpu_qwen3.h).
//
// Reference: qwen3/main.cpp:118-329 (Engine) and :17-102,333-363 (command
// line); checkpoint validation qwen3/model.cpp:376-495. The reference engine
// issues 14 synchronising launches per layer (main.cpp:159-226); the default
// mode here runs 5 fused kernels per layer plus 2 for the logits/argmax,
// captured once into a HIP graph whose decode position and token live in
// device memory, so a whole prompt + generation runs without host round
// trips. XPU_QWEN3_REFERENCE keeps the reference's kernel sequence.
//
// Memory layout (one arena, 4 KiB aligned tensors as in model.cpp:481-491):
// per layer [q; k; v] projection (rows q then k then v), o_proj, [gate; up]
// (2I x H), down_proj, the four norm gains; then embed_tokens, the final norm
// and, when untied, lm_head. KV caches bf16: K and V chunk-major
// [layer][kv_head][16][max_seq][8] (the reference-mode kernels use
// [layer][max_seq][kv_head][128] for both).
#include "../../include/xpu_qwen3.h"
#include "../../include/xpu_kernels.h"
#include "host_common.hpp"
#include "json.hpp"
#include "runtime_internal.hpp"

#include <algorithm>
#include <chrono>
#include <map>
#include <cstdlib>
#include <cstdio>
#include <fstream>
#include <iostream>
#include <set>
#include <sstream>
#include <thread>

using xpu::set_error;

namespace {

constexpr uint32_t kEos = 151645, kEndOfTurn = 151643;  // qwen3/model.hpp:19-20
constexpr uint32_t kMaxContext = 40960;                 // qwen3/model.hpp:18
constexpr uint32_t kTensorKinds = 14;                   // XPU_W_* plus lm_head (13)
constexpr int kLmHead = XPU_W_LMHEAD;


uint64_t tensor_elems(const xpu_qwen3_config &c, int kind) {
  const uint64_t h = c.hidden, qd = uint64_t{c.heads} * c.head_dim, kvd = uint64_t{c.kv_heads} * c.head_dim,
                 in = c.intermediate;
  switch (kind) {
    case XPU_W_Q: return qd * h;
    case XPU_W_K: case XPU_W_V: return kvd * h;
    case XPU_W_O: return h * qd;
    case XPU_W_QNORM: case XPU_W_KNORM: return c.head_dim;
    case XPU_W_GATE: case XPU_W_UP: return in * h;
    case XPU_W_DOWN: return h * in;
    case XPU_W_INNORM: case XPU_W_POSTNORM: case XPU_W_FINALNORM: return h;
    case XPU_W_EMBED: case kLmHead: return uint64_t{c.vocab} * h;
    default: return 0;
  }
}

bool is_gain(int kind) {
  return kind == XPU_W_QNORM || kind == XPU_W_KNORM || kind == XPU_W_INNORM || kind == XPU_W_POSTNORM ||
         kind == XPU_W_FINALNORM;
}

uint64_t tensor_seed(uint64_t seed, int kind, uint32_t layer) {
  return xpu::mix64(seed ^ (0x51ed270b27e5a3c1ull * static_cast<uint64_t>(kind + 1)) ^
                    (0x2545f4914f6cdd1dull * static_cast<uint64_t>(layer + 1)));
}

template <typename F> void parallel_for(uint64_t n, F f) {
  const unsigned threads = std::max(1u, std::min(32u, std::thread::hardware_concurrency()));
  if (n < (1u << 16) || threads == 1) {
    f(0, n);
    return;
  }
  std::vector<std::thread> pool;
  const uint64_t per = (n + threads - 1) / threads;
  for (unsigned t = 0; t < threads; ++t) {
    const uint64_t b = t * per, e = std::min(n, b + per);
    if (b < e) pool.emplace_back(f, b, e);
  }
  for (auto &th : pool) th.join();
}

void fill_tensor(const xpu_qwen3_config &c, uint64_t seed, float gain_std, int kind, uint32_t layer,
                 uint16_t *out) {
  const uint64_t n = tensor_elems(c, kind);
  const uint64_t ts = tensor_seed(seed, kind, layer);
  if (is_gain(kind)) {
    for (uint64_t i = 0; i < n; ++i)
      out[i] = xpu::f32_to_bf16(gain_std == 0.0f ? 1.0f
                                                 : static_cast<float>(1.0 + xpu::normal_from_hash(
                                                                                xpu::counter_hash(ts, i)) *
                                                                                static_cast<double>(gain_std)));
    return;
  }
  parallel_for(n, [&](uint64_t b, uint64_t e) {
    for (uint64_t i = b; i < e; ++i)
      out[i] = xpu::f32_to_bf16(
          static_cast<float>(xpu::normal_from_hash(xpu::counter_hash(ts, i)) * static_cast<double>(0.02f)));
  });
}

int validate_config(const xpu_qwen3_config &c) {
  if (c.head_dim != 128) return set_error(XPU_ERR_INVALID, "Qwen3 kernels need head_dim 128");
  if (!c.hidden || !c.intermediate || !c.layers || !c.heads || !c.kv_heads || !c.vocab)
    return set_error(XPU_ERR_INVALID, "Qwen3 config has a zero dimension");
  if (c.heads % c.kv_heads) return set_error(XPU_ERR_INVALID, "heads must be a multiple of kv_heads");
  if (c.hidden % 8 || c.intermediate % 8)
    return set_error(XPU_ERR_INVALID, "hidden and intermediate sizes must be multiples of 8");
  if (c.hidden > 16384 || c.intermediate > 65536 || c.heads * c.head_dim > 32768)
    return set_error(XPU_ERR_INVALID, "Qwen3 config exceeds the kernels' LDS-staged vector sizes");
  return XPU_OK;
}

struct Layer {
  uint16_t *qkv, *o, *gu, *down, *in_norm, *post_norm, *q_norm, *k_norm;
};

uint64_t align4k(uint64_t v) { return (v + 4095) & ~uint64_t{4095}; }
uint32_t kpad_bytes(uint32_t k) { return ((k + 511u) & ~511u) * 2u; }

}  // namespace

struct xpu_qwen3 {
  xpu_runtime *rt = nullptr;
  bool owns_rt = false;
  xpu_qwen3_config c{};
  uint32_t max_seq = 0;
  int mode = XPU_QWEN3_GRAPH;
  // layout of the positions held in the KV caches: -1 none written yet,
  // 0 chunk-major (graph and eager modes), 1 position-major (reference mode)
  int kv_layout = -1;
  uint8_t *arena = nullptr;
  uint64_t arena_bytes = 0;
  std::vector<Layer> layers;
  uint16_t *embed = nullptr, *final_norm = nullptr, *lm_head = nullptr;
  uint16_t *kcache = nullptr, *vcache = nullptr, *cos_t = nullptr, *sin_t = nullptr;
  uint16_t *x = nullptr, *qkv = nullptr, *attn = nullptr, *h = nullptr, *up = nullptr, *logits = nullptr;
  uint16_t *norm = nullptr, *tmp = nullptr;
  uint16_t *rope_row = nullptr;  // cos and sin rows of the decode position state[0]
  float *part_val = nullptr;
  uint32_t *part_idx = nullptr, *part_bad = nullptr, *state = nullptr, *prompt = nullptr, *gen = nullptr;
  uint32_t *ref_token = nullptr;
  uint32_t nparts = 0;
  void *graph = nullptr;
  // attention split over compute units (xpu_q3_attn_scores + xpu_q3_attn_pv)
  // for contexts of at least split_from positions (0: never), with its own
  // graph; scores [heads][att_spitch] and maxima [heads][att_parts]
  bool split_ok = false;
  // the attention kernel's spare blocks prefetch the layer's o_proj,
  // [gate; up] and down_proj only when they fit well inside the Infinity
  // Cache (setup_launches)
  bool attn_prefetch = false;
  uint32_t split_from = 257, att_spitch = 0, att_parts = 0;
  float *att_scores = nullptr, *att_max = nullptr;
  void *graph_split = nullptr;
  // fused-path geometry
  struct Launch {
    const xpu::KernelInfo *k = nullptr;
    uint32_t grid = 0, shared = 0;
  } qkv_l, attn_l, scores_l, pv_l, o_l, gu_l, down_l, logits_l, finish_l;
  // batched prefill (kernels/qwen3_ops.hip part 3): chunk buffers of
  // pf_chunk tokens; pf_ok when the shape has kernels for every projection;
  // gemm_prefill: the projections on the MFMA GEMM (pf_gemm_ok when the
  // module has its kernels)
  bool pf_ok = false, batched_prefill = false, pf_gemm_ok = false, gemm_prefill = false;
  uint32_t pf_chunk = 0, pf_chunk_gemm = 0;
  // the prompt buffers are sized for the batched form's chunks at creation
  // and grow to the GEMM form's (and its [T][2I] buffer) when that form is
  // selected: pf_rows token rows, pf_gemm_sized with the [gate | up] buffer
  uint64_t pf_rows = 0;
  bool pf_gemm_sized = false;
  void *pf_block = nullptr;
  uint16_t *pf_x = nullptr, *pf_xn = nullptr, *pf_qkv = nullptr, *pf_q = nullptr, *pf_a = nullptr,
           *pf_h = nullptr, *pf_gu = nullptr;
  const xpu::KernelInfo *pf_silu_k = nullptr, *pf_attn_mfma_k = nullptr;
  const xpu::KernelInfo *pf_attn_short_k = nullptr;  // chunks whose contexts stay within 256 positions
  const xpu::KernelInfo *pf_embed_k = nullptr, *pf_norm_k = nullptr, *pf_rope_k = nullptr, *pf_attn_k = nullptr,
                        *pf_qkv_k = nullptr, *pf_o_k = nullptr, *pf_gu_k = nullptr, *pf_down_k = nullptr;
  // rows per wavefront of those four batched GEMV kernels (their _r<R>)
  uint32_t pf_qkv_r = 0, pf_o_r = 0, pf_gu_r = 0, pf_down_r = 0;

  ~xpu_qwen3() {
    if (graph) xpu_rt_graph_destroy(graph);
    if (graph_split) xpu_rt_graph_destroy(graph_split);
    if (rt) {
      for (void *p : {static_cast<void *>(arena), static_cast<void *>(kcache), static_cast<void *>(vcache),
                      static_cast<void *>(cos_t), static_cast<void *>(sin_t), static_cast<void *>(x), pf_block})
        if (p) xpu_rt_free(rt, p);
      if (owns_rt) xpu_rt_destroy(rt);
    }
  }
};

namespace {

// Activation block: one allocation, 256-byte aligned sub-buffers.
int allocate_buffers(xpu_qwen3 &e) {
  const xpu_qwen3_config &c = e.c;
  const uint64_t qd = uint64_t{c.heads} * c.head_dim, kvd = uint64_t{c.kv_heads} * c.head_dim;
  const uint64_t cache = uint64_t{c.layers} * c.kv_heads * e.max_seq * c.head_dim * 2;
  const uint64_t rope = uint64_t{e.max_seq} * c.head_dim * 2;
  e.nparts = e.rt->compute_units * 8;
  e.att_parts = std::min(64u, std::max(1u, e.rt->compute_units / c.heads));
  e.att_spitch = (e.max_seq + 511u) & ~511u;
  std::vector<std::pair<void **, uint64_t>> parts = {
      {reinterpret_cast<void **>(&e.x), c.hidden * 2ull},
      {reinterpret_cast<void **>(&e.qkv), (qd + 2 * kvd) * 2},
      {reinterpret_cast<void **>(&e.attn), qd * 2},
      {reinterpret_cast<void **>(&e.h), c.intermediate * 2ull},
      {reinterpret_cast<void **>(&e.up), c.intermediate * 2ull},
      {reinterpret_cast<void **>(&e.logits), c.vocab * 2ull},
      {reinterpret_cast<void **>(&e.norm), c.hidden * 2ull},
      {reinterpret_cast<void **>(&e.tmp), std::max<uint64_t>(c.hidden, qd) * 2},
      {reinterpret_cast<void **>(&e.part_val), e.nparts * 4ull},
      {reinterpret_cast<void **>(&e.part_idx), e.nparts * 4ull},
      {reinterpret_cast<void **>(&e.part_bad), e.nparts * 4ull},
      {reinterpret_cast<void **>(&e.state), 64},
      {reinterpret_cast<void **>(&e.rope_row), 2ull * c.head_dim * 2},
      {reinterpret_cast<void **>(&e.prompt), e.max_seq * 4ull},
      {reinterpret_cast<void **>(&e.gen), e.max_seq * 4ull},
      {reinterpret_cast<void **>(&e.ref_token), 4},
      {reinterpret_cast<void **>(&e.att_scores), uint64_t{c.heads} * e.att_spitch * 4},
      {reinterpret_cast<void **>(&e.att_max), uint64_t{c.heads} * e.att_parts * 4},
  };
  uint64_t total = 0;
  for (auto &p : parts) total += (p.second + 255) & ~uint64_t{255};
  int rc = xpu_rt_require_device_and_memory(e.rt, e.arena_bytes + 2 * cache + 2 * rope + total);
  if (rc) return rc;
  void *block = nullptr;
  if ((rc = xpu_rt_alloc(e.rt, e.arena_bytes, 4096, reinterpret_cast<void **>(&e.arena)))) return rc;
  if ((rc = xpu_rt_alloc(e.rt, cache, 4096, reinterpret_cast<void **>(&e.kcache)))) return rc;
  if ((rc = xpu_rt_alloc(e.rt, cache, 4096, reinterpret_cast<void **>(&e.vcache)))) return rc;
  if ((rc = xpu_rt_alloc(e.rt, rope, 4096, reinterpret_cast<void **>(&e.cos_t)))) return rc;
  if ((rc = xpu_rt_alloc(e.rt, rope, 4096, reinterpret_cast<void **>(&e.sin_t)))) return rc;
  if ((rc = xpu_rt_alloc(e.rt, total, 4096, &block))) return rc;
  uint8_t *p = static_cast<uint8_t *>(block);
  for (auto &part : parts) {
    *part.first = p;
    p += (part.second + 255) & ~uint64_t{255};
  }
  if ((rc = xpu_rt_memset(e.rt, block, 0, total))) return rc;
  if ((rc = xpu_rt_memset(e.rt, e.kcache, 0, cache))) return rc;
  if ((rc = xpu_rt_memset(e.rt, e.vcache, 0, cache))) return rc;
  // RoPE tables (main.cpp:299-318)
  std::vector<uint16_t> cs(uint64_t{e.max_seq} * c.head_dim), sn(cs.size());
  xpu_qwen3_rope_tables(cs.data(), sn.data(), e.max_seq, c.head_dim, c.rope_theta);
  if ((rc = xpu_rt_copy_to_device(e.rt, e.cos_t, cs.data(), rope))) return rc;
  return xpu_rt_copy_to_device(e.rt, e.sin_t, sn.data(), rope);
}

// Arena plan: pointers of every tensor inside the weight arena.
void plan_arena(xpu_qwen3 &e, uint8_t *base) {
  const xpu_qwen3_config &c = e.c;
  const uint64_t H = c.hidden, qd = uint64_t{c.heads} * c.head_dim, kvd = uint64_t{c.kv_heads} * c.head_dim,
                 I = c.intermediate;
  uint64_t off = 0;
  auto take = [&](uint64_t elems) {
    uint16_t *p = reinterpret_cast<uint16_t *>(base + off);
    off = align4k(off + elems * 2);
    return p;
  };
  e.layers.resize(c.layers);
  for (auto &L : e.layers) {
    L.qkv = take((qd + 2 * kvd) * H);
    L.o = take(H * qd);
    L.gu = take(2 * I * H);
    L.down = take(H * I);
    L.in_norm = take(H);
    L.post_norm = take(H);
    L.q_norm = take(c.head_dim);
    L.k_norm = take(c.head_dim);
  }
  e.embed = take(uint64_t{c.vocab} * H);
  e.final_norm = take(H);
  e.lm_head = c.tied ? e.embed : take(uint64_t{c.vocab} * H);
  e.arena_bytes = off;
}

// Device location of a logical tensor (the q/k/v and gate/up parts sit
// inside the fused matrices).
uint16_t *tensor_location(xpu_qwen3 &e, int kind, uint32_t layer) {
  const xpu_qwen3_config &c = e.c;
  const uint64_t H = c.hidden, qd = uint64_t{c.heads} * c.head_dim, kvd = uint64_t{c.kv_heads} * c.head_dim;
  if (kind == XPU_W_EMBED) return e.embed;
  if (kind == XPU_W_FINALNORM) return e.final_norm;
  if (kind == kLmHead) return e.lm_head;
  Layer &L = e.layers[layer];
  switch (kind) {
    case XPU_W_Q: return L.qkv;
    case XPU_W_K: return L.qkv + qd * H;
    case XPU_W_V: return L.qkv + (qd + kvd) * H;
    case XPU_W_O: return L.o;
    case XPU_W_QNORM: return L.q_norm;
    case XPU_W_KNORM: return L.k_norm;
    case XPU_W_GATE: return L.gu;
    case XPU_W_UP: return L.gu + uint64_t{c.intermediate} * H;
    case XPU_W_DOWN: return L.down;
    case XPU_W_INNORM: return L.in_norm;
    case XPU_W_POSTNORM: return L.post_norm;
    default: return nullptr;
  }
}

int setup_launches(xpu_qwen3 &e) {
  const xpu_qwen3_config &c = e.c;
  // at most 4 blocks per CU for the decode GEMVs (Qwen3-0.6B: 2 measured
  // the same, 1 slower); 2 for matrices past 32 MB (Qwen3-8B: 311 -> 320
  // tok/s, 1 slower)
  const uint32_t cap = e.rt->compute_units * 4;
  auto cap_for = [&](uint64_t rows, uint64_t K) {
    return rows * K * 2 > (32ull << 20) ? e.rt->compute_units * 2 : cap;
  };
  auto find = [&](const char *name, xpu_qwen3::Launch &l) -> int {
    l.k = e.rt->find_exact(name);
    return l.k ? XPU_OK : set_error(XPU_ERR_NOT_FOUND, std::string("kernel is absent from module: ") + name);
  };
  const uint32_t qkv_rows = (c.heads + 2 * c.kv_heads) * c.head_dim, qd = c.heads * c.head_dim;
  int rc;
  // Register-vector kernels (_v<NC>: vector slices and RMSNorm in lane
  // registers, no LDS) when K <= 512 NC for a built NC; else the LDS-staged
  // kernels.
  auto reg_nc = [](uint32_t K) -> uint32_t {
    for (uint32_t nc : {1u, 2u, 4u, 6u, 8u})
      if (K <= 512u * nc) return nc;
    return 0;
  };
  auto pick = [&](const std::string &reg_base, uint32_t K, const char *lds_name, xpu_qwen3::Launch &l) -> int {
    const uint32_t nc = reg_nc(K);
    if (nc) {
      l.k = e.rt->find_exact(reg_base + "_v" + std::to_string(nc));
      l.shared = 0;
      if (l.k) return XPU_OK;
    }
    l.shared = kpad_bytes(K);
    return find(lds_name, l);
  };
  if ((rc = pick("xpu_q3_norm_gemv_r2", c.hidden, "xpu_q3_norm_gemv_r2", e.qkv_l))) return rc;
  e.qkv_l.grid = std::min(cap_for(qkv_rows, c.hidden), (qkv_rows + 7) / 8);
  if ((rc = find("xpu_q3_attention", e.attn_l))) return rc;
  // One block per query head; the other compute units prefetch the layer's
  // remaining weights into the 256 MiB Infinity Cache, for the kernels that
  // follow, when those fit in a quarter of it (Qwen3-0.6B: 23 MB). Larger
  // layers (Qwen3-8B: 335 MB) would stream through the cache and evict
  // themselves before use; their attention runs without spare blocks.
  {
    const uint64_t qd = uint64_t{c.heads} * c.head_dim, rest = uint64_t{c.hidden} * (qd + 3ull * c.intermediate) * 2;
    constexpr uint64_t kPrefetchBudget = 64ull << 20;
    e.attn_prefetch = rest <= kPrefetchBudget;
  }
  e.attn_l.grid = e.attn_prefetch ? std::max(c.heads, e.rt->compute_units) : c.heads;
  e.scores_l.k = e.rt->find_exact("xpu_q3_attn_scores");
  e.pv_l.k = e.rt->find_exact("xpu_q3_attn_pv");
  e.scores_l.grid = c.heads * e.att_parts;
  e.pv_l.grid = c.heads * 8;  // 16 output dims per block
  // probabilities (4096 floats) + V rows (4096 x 16 codes) of a softmax
  // chunk + 64 chunk sums + 4 x 16 wave partials
  e.pv_l.shared = 4096 * 4 + 4096 * 16 * 2 + 64 * 4 + 64 * 4;
  e.split_ok = e.scores_l.k && e.pv_l.k && e.max_seq <= 64u * 4096u && e.pv_l.shared <= e.rt->max_shared;
  if ((rc = pick("xpu_q3_gemv_residual_r1", qd, "xpu_q3_gemv_residual_r1", e.o_l))) return rc;
  e.o_l.grid = std::min(cap_for(c.hidden, qd), (c.hidden + 3) / 4);
  if ((rc = pick("xpu_q3_norm_gemv_swiglu_r2", c.hidden, "xpu_q3_norm_gemv_swiglu_r2", e.gu_l))) return rc;
  e.gu_l.grid = std::min(cap_for(2ull * c.intermediate, c.hidden), (c.intermediate + 3) / 4);
  if ((rc = pick("xpu_q3_gemv_residual_r1", c.intermediate, "xpu_q3_gemv_residual_r1", e.down_l))) return rc;
  e.down_l.grid = std::min(cap_for(c.hidden, c.intermediate), (c.hidden + 3) / 4);
  if ((rc = pick("xpu_q3_norm_gemv_logits_r2", c.hidden, "xpu_q3_norm_gemv_logits_r2", e.logits_l))) return rc;
  // two blocks per CU: 8 MiB of lm_head rows in flight on 256 CUs, the
  // streaming optimum (8 blocks per CU, or a second row buffer per
  // wavefront, read slower)
  e.logits_l.grid = std::min(std::min(e.nparts, e.rt->compute_units * 2), (c.vocab + 7) / 8);
  if ((rc = find("xpu_q3_argmax_finish", e.finish_l))) return rc;
  e.finish_l.grid = 1;
  for (auto *l : {&e.qkv_l, &e.o_l, &e.gu_l, &e.down_l, &e.logits_l})
    if (l->shared > e.rt->max_shared) return set_error(XPU_ERR_INVALID, "Qwen3 vector exceeds the LDS");
  return XPU_OK;
}

// The batched GEMV form needs every projection's K to be 512 times a chunk
// count the module has kernels for (xpu_q3_pf_gemv_e<epi>_c<K/512>); the
// GEMM form needs none of those. The two share the embedding, RMSNorm and
// QK-norm/RoPE/cache kernels and the chunk buffers.
// The prompt chunk buffers for the batched form (gemm = false: pf_chunk
// rows) or the GEMM form (pf_chunk_gemm rows plus the [T][2I] [gate | up]
// output, and the GEMM's split-K partials reserved in the runtime's
// workspace so that no prompt grows it mid-way): the residual stream X and
// its normed copy [T][H], the QKV output [T][(Hq+2Hkv)·128], the roped
// queries and the attention output [T][Hq·128], the SwiGLU output [T][I].
// Grows only; the GEMM form's buffers serve the batched form too.
int size_prompt_buffers(xpu_qwen3 &e, bool gemm) {
  const xpu_qwen3_config &c = e.c;
  const uint64_t T = gemm ? e.pf_chunk_gemm : e.pf_chunk;
  if (T <= e.pf_rows && (!gemm || e.pf_gemm_sized)) return XPU_OK;
  const uint64_t qd = uint64_t{c.heads} * c.head_dim;
  const uint64_t qkv_rows = uint64_t{c.heads + 2 * c.kv_heads} * c.head_dim;
  const uint64_t sizes[7] = {T * c.hidden, T * c.hidden, T * qkv_rows, T * qd, T * qd, T * c.intermediate,
                             gemm ? T * 2 * c.intermediate : 0};
  uint64_t total = 0;
  for (uint64_t n : sizes) total += (n * 2 + 255) & ~uint64_t{255};
  int rc;
  if (e.pf_block) {
    if ((rc = xpu_rt_free(e.rt, e.pf_block))) return rc;  // waits for the stream first
    e.pf_block = nullptr;
    e.pf_rows = 0;
    e.pf_gemm_sized = false;
  }
  if ((rc = xpu_rt_alloc(e.rt, total, 4096, &e.pf_block))) return rc;
  uint16_t **dst[7] = {&e.pf_x, &e.pf_xn, &e.pf_qkv, &e.pf_q, &e.pf_a, &e.pf_h, &e.pf_gu};
  uint8_t *p = static_cast<uint8_t *>(e.pf_block);
  for (int i = 0; i < 7; ++i) {
    *dst[i] = sizes[i] ? reinterpret_cast<uint16_t *>(p) : nullptr;
    p += (sizes[i] * 2 + 255) & ~uint64_t{255};
  }
  e.pf_rows = T;
  e.pf_gemm_sized = gemm;
  if (gemm) {
    void *ws = nullptr;
    if ((rc = e.rt->scratch(xpu::gemm_nt_workspace_bound(e.rt), &ws))) return rc;
  }
  return XPU_OK;
}

int setup_prefill(xpu_qwen3 &e) {
  const xpu_qwen3_config &c = e.c;
  const uint32_t qd = c.heads * c.head_dim;
  // the kernel with the most rows per wavefront the module has
  auto gemv = [&](int epi, uint32_t K, uint32_t &r) -> const xpu::KernelInfo * {
    if (K % 512u) return nullptr;
    for (uint32_t rows : {4u, 2u, 1u}) {
      const xpu::KernelInfo *k = e.rt->find_exact("xpu_q3_pf_gemv_e" + std::to_string(epi) + "_c" +
                                                  std::to_string(K / 512u) + "_r" + std::to_string(rows));
      if (k) {
        r = rows;
        return k;
      }
    }
    return nullptr;
  };
  e.pf_qkv_k = gemv(0, c.hidden, e.pf_qkv_r);
  e.pf_o_k = gemv(1, qd, e.pf_o_r);
  e.pf_gu_k = gemv(2, c.hidden, e.pf_gu_r);
  e.pf_down_k = gemv(1, c.intermediate, e.pf_down_r);
  e.pf_embed_k = e.rt->find_exact("xpu_q3_pf_embed");
  e.pf_norm_k = e.rt->find_exact("xpu_q3_pf_rmsnorm");
  e.pf_rope_k = e.rt->find_exact("xpu_q3_pf_rope_cache");
  e.pf_attn_k = e.rt->find_exact("xpu_q3_pf_attention");
  e.pf_attn_short_k = e.rt->find_exact("xpu_q3_pf_attention_short");
  const bool common = e.pf_embed_k && e.pf_norm_k && e.pf_rope_k && c.hidden % 8 == 0;
  e.pf_ok = common && e.pf_qkv_k && e.pf_o_k && e.pf_gu_k && e.pf_down_k && e.pf_attn_k &&
            [&] {
              // the batched GEMVs' LDS: two tiles of 8 token rows for K <= 2048, one past that
              for (uint32_t K : {c.hidden, qd, c.intermediate})
                if ((K <= 2048u ? 2u : 1u) * 16u * K > e.rt->max_shared) return false;
              return true;
            }();
  const uint64_t qkv_rows = uint64_t{c.heads + 2 * c.kv_heads} * c.head_dim;
  // the MFMA form: every projection's K and N multiples of 8 (the NT GEMM
  // kernels read the weight rows in place) and 1, 2 or 4 query heads per kv
  // head (the MFMA attention's 128 query rows per block)
  const uint32_t group = c.heads / c.kv_heads;
  e.pf_silu_k = e.rt->find_exact("xpu_q3_pf_silu_mul");
  if (group == 1 || group == 2 || group == 4)
    e.pf_attn_mfma_k = e.rt->find_exact("xpu_q3_pf_attention_mfma_g" + std::to_string(group));
  e.pf_gemm_ok = common && e.pf_silu_k && e.pf_attn_mfma_k && e.rt->find_exact("xpu_gemm_bf16_nt_dma") &&
                 c.intermediate % 8 == 0 && qd % 8 == 0 && qkv_rows % 8 == 0;
  if (!e.pf_ok && !e.pf_gemm_ok) return XPU_OK;
  // chunks of 256 positions for the batched GEMV form; up to 4096 for the
  // GEMM form, whose GEMMs and attention fill the chip only with long chunks
  e.pf_chunk = e.pf_ok ? std::min<uint32_t>(e.max_seq, 256) : 0;
  e.pf_chunk_gemm = e.pf_gemm_ok ? std::min<uint32_t>(e.max_seq, 4096) : 0;
  e.batched_prefill = e.pf_ok;  // the default: the bit-identical form; the GEMM form is opt-in
  return e.pf_ok ? size_prompt_buffers(e, false) : XPU_OK;
}

int launch(xpu_qwen3 &e, const xpu_qwen3::Launch &l, uint32_t block, std::initializer_list<xpu_kernel_arg> args) {
  return e.rt->launch(*l.k, l.grid, 1, block, l.shared, args.begin(), static_cast<uint32_t>(args.size()));
}

// o_proj + residual, RMSNorm + [gate; up] + SiLU, down + residual of layer
// L for the residual stream in e.x, from the attention output `attn`.
int enqueue_layer_mlp(xpu_qwen3 &e, const Layer &L, const uint16_t *attn) {
  const xpu_qwen3_config &c = e.c;
  const uint32_t H = c.hidden, I = c.intermediate, qd = c.heads * c.head_dim;
  const float eps = c.rms_eps;
  int rc;
  if ((rc = launch(e, e.o_l, 256, {{8, &L.o}, {8, &attn}, {8, &e.x}, {4, &H}, {4, &qd}}))) return rc;
  if ((rc = launch(e, e.gu_l, 256,
                   {{8, &L.gu}, {8, &e.x}, {8, &L.post_norm}, {8, &e.h}, {4, &I}, {4, &H}, {4, &eps}})))
    return rc;
  return launch(e, e.down_l, 256, {{8, &L.down}, {8, &e.h}, {8, &e.x}, {4, &H}, {4, &I}});
}

// Final RMSNorm + lm_head + argmax of e.x; the finish kernel stores the
// token and advances state (position, token, RoPE rows).
int enqueue_head(xpu_qwen3 &e) {
  const xpu_qwen3_config &c = e.c;
  const uint32_t H = c.hidden, V = c.vocab, max_seq = e.max_seq;
  const float eps = c.rms_eps;
  int rc;
  if ((rc = launch(e, e.logits_l, 256,
                   {{8, &e.lm_head}, {8, &e.x}, {8, &e.final_norm}, {8, &e.logits}, {4, &V}, {4, &H}, {4, &eps},
                    {8, &e.part_val}, {8, &e.part_idx}, {8, &e.part_bad}})))
    return rc;
  const uint32_t nparts = e.logits_l.grid;
  return launch(e, e.finish_l, 1024,
                {{8, &e.part_val}, {8, &e.part_idx}, {8, &e.part_bad}, {4, &nparts}, {8, &e.state},
                 {8, &e.prompt}, {8, &e.gen}, {4, &max_seq}, {8, &e.cos_t}, {8, &e.sin_t}, {8, &e.rope_row},
                 {4, &max_seq}});
}

// One token through the fused kernels (reads position/token from state).
int enqueue_fused_step(xpu_qwen3 &e, bool split) {
  const xpu_qwen3_config &c = e.c;
  const uint32_t H = c.hidden, I = c.intermediate, V = c.vocab, heads = c.heads, kv = c.kv_heads;
  const uint32_t qkv_rows = (heads + 2 * kv) * c.head_dim, max_seq = e.max_seq;
  const float eps = c.rms_eps;
  const float scale = static_cast<float>(1.0 / std::sqrt(static_cast<double>(c.head_dim)));
  const uint64_t cache_layer = uint64_t{kv} * max_seq * c.head_dim;
  const uint16_t *no_embed = nullptr;
  const uint16_t *sin_row = e.rope_row + c.head_dim;
  int rc;
  for (uint32_t l = 0; l < c.layers; ++l) {
    const Layer &L = e.layers[l];
    const uint16_t *embed = l == 0 ? e.embed : no_embed;
    uint16_t *kc = e.kcache + l * cache_layer, *vc = e.vcache + l * cache_layer;
    if ((rc = launch(e, e.qkv_l, 256,
                     {{8, &L.qkv}, {8, &e.x}, {8, &L.in_norm}, {8, &e.qkv}, {4, &qkv_rows}, {4, &H}, {4, &eps},
                      {8, &embed}, {8, &e.state}, {4, &V}})))
      return rc;
    // the attention kernel's spare blocks prefetch this layer's o_proj,
    // [gate; up] and down_proj (contiguous in the arena)
    const uint16_t *pf = L.o;
    const uint8_t *pf_end = reinterpret_cast<const uint8_t *>(L.down) + uint64_t{H} * I * 2;
    const uint64_t pf_bytes =
        e.attn_prefetch ? static_cast<uint64_t>(pf_end - reinterpret_cast<const uint8_t *>(L.o)) : 0;
    const uint32_t pf_delay = 1;  // the spare blocks start ~512 cycles after the attention's loads
    if (split) {
      const uint32_t spitch = e.att_spitch, parts = e.att_parts;
      if ((rc = launch(e, e.scores_l, 256,
                       {{8, &e.qkv}, {8, &L.q_norm}, {8, &L.k_norm}, {8, &e.rope_row}, {8, &sin_row}, {8, &kc},
                        {8, &vc}, {8, &e.att_scores}, {8, &e.att_max}, {8, &e.state}, {4, &heads}, {4, &kv},
                        {4, &max_seq}, {4, &spitch}, {4, &parts}, {4, &eps}, {4, &scale}})))
        return rc;
      if ((rc = launch(e, e.pv_l, 256,
                       {{8, &e.att_scores}, {8, &e.att_max}, {8, &vc}, {8, &e.attn}, {8, &e.state}, {4, &heads},
                        {4, &kv}, {4, &max_seq}, {4, &spitch}, {4, &parts}})))
        return rc;
    } else if ((rc = launch(e, e.attn_l, 256,
                     {{8, &e.qkv}, {8, &L.q_norm}, {8, &L.k_norm}, {8, &e.rope_row}, {8, &sin_row}, {8, &kc},
                      {8, &vc}, {8, &e.attn}, {8, &e.state}, {4, &heads}, {4, &kv}, {4, &max_seq}, {4, &eps},
                      {4, &scale}, {8, &pf}, {8, &pf_bytes}, {4, &pf_delay}})))
      return rc;
    if ((rc = enqueue_layer_mlp(e, L, e.attn))) return rc;
  }
  return enqueue_head(e);
}

// K/V cache entries of prompt positions [0, P) (prompt ids already in
// e.prompt), in chunks of pf_chunk positions (pf_chunk_gemm in the GEMM
// form). The last layer's o_proj and MLP are skipped: only the caches are
// wanted. With `head`, position P - 1 also yields the next token: its row of
// the residual stream goes to e.x and the decode step's kernels finish it
// (the last layer's o_proj and MLP, then the final norm, lm_head and argmax
// with state[0] = P - 1), so no separate decode step runs for it.
int run_prefill(xpu_qwen3 &e, uint32_t P, bool head) {
  const xpu_qwen3_config &c = e.c;
  uint32_t H = c.hidden, I = c.intermediate, V = c.vocab, heads = c.heads, kv = c.kv_heads, max_seq = e.max_seq;
  uint32_t qkv_rows = (heads + 2 * kv) * c.head_dim, qd = heads * c.head_dim;
  float eps = c.rms_eps;
  // two tiles of 8 token rows of K codes (xpu_q3_pf_gemv_*)
  // LDS of the batched GEMVs: two tiles of 8 token rows for K <= 2048, one
  // past that
  auto pf_lds = [](uint32_t K) { return (K <= 2048u ? 2u : 1u) * 8u * K * 2u; };
  float scale = static_cast<float>(1.0 / std::sqrt(static_cast<double>(c.head_dim)));
  const uint64_t cache_layer = uint64_t{kv} * max_seq * c.head_dim;
  xpu_runtime *rt = e.rt;
  auto go = [&](const xpu::KernelInfo *k, uint32_t gx, uint32_t gy, uint32_t block, uint32_t shared,
                std::initializer_list<xpu_kernel_arg> args) {
    return rt->launch(*k, gx, gy, block, shared, args.begin(), static_cast<uint32_t>(args.size()));
  };
  int rc;
  const uint32_t chunk = e.gemm_prefill ? e.pf_chunk_gemm : e.pf_chunk;
  for (uint32_t p0 = 0; p0 < P; p0 += chunk) {
    uint32_t T = std::min(chunk, P - p0);
    // batched GEMV grids: 4 wavefronts of R rows (R / 2 output pairs for
    // [gate; up]) per block; past one token tile, the tokens split into
    // R / 2 groups (R for the residual forms), which keeps the block count
    // of 2-row (1-row) wavefronts over all tokens, times the factor at each
    // launch that fills the blocks per compute unit its registers and LDS
    // allow (measured: QKV and [gate; up] 3/2, o_proj 2, down_proj 2)
    auto groups = [&](uint32_t r, uint32_t base) { return T > 8 ? std::max(1u, r / base) : 1u; };
    if ((rc = go(e.pf_embed_k, T, 1, 256, 0, {{8, &e.embed}, {8, &e.prompt}, {4, &p0}, {8, &e.pf_x}, {4, &H}, {4, &V}})))
      return rc;
    // the GEMM form's split-K reductions of o_proj and down_proj can write
    // the RMSNorm that follows them (xn_ready: pf_xn holds this layer's
    // normalised input)
    bool xn_ready = false;
    for (uint32_t l = 0; l < c.layers; ++l) {
      const Layer &L = e.layers[l];
      uint16_t *kc = e.kcache + l * cache_layer, *vc = e.vcache + l * cache_layer;
      if (!xn_ready && (rc = go(e.pf_norm_k, (T + 3) / 4, 1, 256, 0,
                                {{8, &e.pf_x}, {8, &L.in_norm}, {8, &e.pf_xn}, {4, &H}, {4, &eps}, {4, &T}})))
        return rc;
      xn_ready = false;
      if (e.gemm_prefill) {
        if ((rc = xpu::gemm_nt(rt, e.pf_xn, L.qkv, e.pf_qkv, T, qkv_rows, H, false))) return rc;
      } else if ((rc = go(e.pf_qkv_k, (qkv_rows + 4 * e.pf_qkv_r - 1) / (4 * e.pf_qkv_r), groups(e.pf_qkv_r, 2) * (T > 8 ? 3u : 2u) / 2u, 256,
                          pf_lds(H),
                          {{8, &L.qkv}, {8, &e.pf_xn}, {8, &e.pf_qkv}, {4, &qkv_rows}, {4, &T}}))) {
        return rc;
      }
      if ((rc = go(e.pf_rope_k, (T + 31) / 32, heads + kv, 256, 0,
                   {{8, &e.pf_qkv}, {8, &L.q_norm}, {8, &L.k_norm}, {8, &e.cos_t}, {8, &e.sin_t}, {8, &kc},
                    {8, &vc}, {8, &e.pf_q}, {4, &p0}, {4, &T}, {4, &heads}, {4, &kv}, {4, &max_seq}, {4, &eps}})))
        return rc;
      if (e.gemm_prefill) {
        // queries per block: 32 U, U = 4 / (G H) with H = 2 key halves for
        // G = 1 and 2, 1 for G = 4
        const uint32_t qrows = heads / kv == 1 ? 64 : 32, blocks = (T + qrows - 1) / qrows * kv;
        if ((rc = go(e.pf_attn_mfma_k, blocks, 1, 256, 0,
                     {{8, &e.pf_q}, {8, &kc}, {8, &vc}, {8, &e.pf_a}, {4, &p0}, {4, &T}, {4, &heads}, {4, &kv},
                      {4, &max_seq}, {4, &scale}})))
          return rc;
      } else {
        const bool short_ctx = e.pf_attn_short_k && p0 + T <= 256;  // every token's context within 256 positions
        if ((rc = go(short_ctx ? e.pf_attn_short_k : e.pf_attn_k, heads, T, 256, 0,
                     {{8, &e.pf_q}, {8, &kc}, {8, &vc}, {8, &e.pf_a}, {4, &p0}, {4, &heads}, {4, &kv},
                      {4, &max_seq}, {4, &scale}})))
          return rc;
      }
      if (l + 1 == c.layers) {
        if (head && p0 + T == P) {
          XPU_HIP_RETURN(hipMemcpyAsync(e.x, e.pf_x + uint64_t{T - 1} * H, uint64_t{H} * 2, hipMemcpyDeviceToDevice,
                                        rt->stream));
          if ((rc = enqueue_layer_mlp(e, L, e.pf_a + uint64_t{T - 1} * qd))) return rc;
          if ((rc = enqueue_head(e))) return rc;
        }
        break;
      }
      bool normed = false;
      if (e.gemm_prefill) {
        if ((rc = xpu::gemm_nt(rt, e.pf_a, L.o, e.pf_x, T, H, qd, true, L.post_norm, e.pf_xn, eps, &normed)))
          return rc;
      } else if ((rc = go(e.pf_o_k, (H + 4 * e.pf_o_r - 1) / (4 * e.pf_o_r), groups(e.pf_o_r, 1) * (T > 8 ? 2u : 1u), 256, pf_lds(qd),
                          {{8, &L.o}, {8, &e.pf_a}, {8, &e.pf_x}, {4, &H}, {4, &T}}))) {
        return rc;
      }
      if (!normed && (rc = go(e.pf_norm_k, (T + 3) / 4, 1, 256, 0,
                              {{8, &e.pf_x}, {8, &L.post_norm}, {8, &e.pf_xn}, {4, &H}, {4, &eps}, {4, &T}})))
        return rc;
      if (e.gemm_prefill) {
        const uint32_t two_i = 2 * I;
        if ((rc = xpu::gemm_nt(rt, e.pf_xn, L.gu, e.pf_gu, T, two_i, H, false))) return rc;
        // 8 columns per thread, 4 tokens per block row
        if ((rc = go(e.pf_silu_k, (I + 2047) / 2048, (T + 3) / 4, 256, 0,
                     {{8, &e.pf_gu}, {8, &e.pf_h}, {4, &I}, {4, &T}})))
          return rc;
        // (the last layer stops after its attention, so layer l + 1 exists)
        if ((rc = xpu::gemm_nt(rt, e.pf_h, L.down, e.pf_x, T, H, I, true, e.layers[l + 1].in_norm, e.pf_xn, eps,
                               &xn_ready)))
          return rc;
        continue;
      }
      if ((rc = go(e.pf_gu_k, (I + 2 * e.pf_gu_r - 1) / (2 * e.pf_gu_r), groups(e.pf_gu_r, 2) * (T > 8 ? 3u : 2u) / 2u,
                   256, pf_lds(H),
                   {{8, &L.gu}, {8, &e.pf_xn}, {8, &e.pf_h}, {4, &I}, {4, &T}})))
        return rc;
      // (one LDS tile past K = 2048: twice the token groups, two blocks per
      // compute unit as its registers allow)
      if ((rc = go(e.pf_down_k, (H + 4 * e.pf_down_r - 1) / (4 * e.pf_down_r),
                   groups(e.pf_down_r, 1) * (I > 2048 && T > 8 ? 2u : 1u), 256,
                   pf_lds(I),
                   {{8, &L.down}, {8, &e.pf_h}, {8, &e.pf_x}, {4, &H}, {4, &T}})))
        return rc;
    }
  }
  return XPU_OK;
}

// The fused step's attention kernels read the RoPE rows of the position in
// e.rope_row; xpu_q3_argmax_finish advances them with the position, and this
// sets them wherever the host writes the position.
int set_rope_row(xpu_qwen3 &e, uint32_t position) {
  const uint64_t hd = e.c.head_dim, at = uint64_t{position} * hd;
  int rc = xpu_rt_copy_device(e.rt, e.rope_row, e.cos_t + at, hd * 2);
  if (!rc) rc = xpu_rt_copy_device(e.rt, e.rope_row + hd, e.sin_t + at, hd * 2);
  return rc;
}

// One decode step at `position` (the value state[0] holds when it runs): the
// attention is split over compute units from split_from positions on; each
// variant has its own graph.
int run_fused_step(xpu_qwen3 &e, uint32_t position) {
  const bool split = e.split_ok && e.split_from && position + 1 >= e.split_from;
  if (e.mode == XPU_QWEN3_EAGER) return enqueue_fused_step(e, split);
  void *&graph = split ? e.graph_split : e.graph;
  if (!graph) {
    int rc = xpu_rt_capture_begin(e.rt);
    if (rc) return rc;
    rc = enqueue_fused_step(e, split);
    void *exec = nullptr;
    const int rc2 = xpu_rt_capture_end(e.rt, &exec);
    if (rc) return rc;
    if (rc2) return rc2;
    graph = exec;
  }
  return xpu_rt_graph_launch(e.rt, graph);
}

// Reference-mode step: the reference's kernel sequence, each launch blocking
// (main.cpp:159-226).
int reference_step(xpu_qwen3 &e, uint32_t token, uint32_t position, uint32_t *next) {
  const xpu_qwen3_config &c = e.c;
  uint32_t H = c.hidden, I = c.intermediate, V = c.vocab, heads = c.heads, kv = c.kv_heads,
           qd = c.heads * c.head_dim, kvd = c.kv_heads * c.head_dim, max_seq = e.max_seq;
  float eps = c.rms_eps;
  uint16_t *q = e.qkv, *k = e.qkv + qd, *v = e.qkv + qd + kvd;
  xpu_runtime *rt = e.rt;
  auto L = [&](const char *name, uint32_t items, std::initializer_list<xpu_kernel_arg> args) {
    return xpu_rt_launch(rt, name, items, args.begin(), static_cast<uint32_t>(args.size()));
  };
  auto rms = [&](uint16_t *in, uint16_t *w, uint16_t *out) {
    return L("QwenRmsNorm", 1, {{8, &in}, {8, &w}, {8, &out}, {4, &H}, {4, &eps}});
  };
  auto gemv = [&](uint16_t *m, uint16_t *vec, uint16_t *out, uint32_t rows, uint32_t cols) {
    return L("QwenGemv", rows, {{8, &m}, {8, &vec}, {8, &out}, {4, &rows}, {4, &cols}});
  };
  int rc;
  if ((rc = L("QwenEmbedding", H, {{8, &e.embed}, {8, &e.x}, {4, &token}, {4, &H}}))) return rc;
  const uint64_t cache_layer = uint64_t{kv} * max_seq * c.head_dim;
  for (uint32_t l = 0; l < c.layers; ++l) {
    Layer &Ly = e.layers[l];
    uint16_t *kc = e.kcache + l * cache_layer, *vc = e.vcache + l * cache_layer;
    if ((rc = rms(e.x, Ly.in_norm, e.norm))) return rc;
    if ((rc = gemv(Ly.qkv, e.norm, q, qd, H))) return rc;
    if ((rc = gemv(Ly.qkv + uint64_t{qd} * H, e.norm, k, kvd, H))) return rc;
    if ((rc = gemv(Ly.qkv + uint64_t{qd + kvd} * H, e.norm, v, kvd, H))) return rc;
    if ((rc = L("QwenQkvRopeCache", heads,
                {{8, &q}, {8, &k}, {8, &v}, {8, &Ly.q_norm}, {8, &Ly.k_norm}, {8, &e.cos_t}, {8, &e.sin_t},
                 {8, &kc}, {8, &vc}, {4, &position}, {4, &max_seq}, {4, &heads}, {4, &kv}})))
      return rc;
    if ((rc = L("QwenAttention", heads,
                {{8, &q}, {8, &kc}, {8, &vc}, {8, &e.attn}, {4, &position}, {4, &heads}, {4, &kv}})))
      return rc;
    if ((rc = gemv(Ly.o, e.attn, e.tmp, H, qd))) return rc;
    if ((rc = L("QwenAdd", H / 32, {{8, &e.x}, {8, &e.tmp}, {4, &H}}))) return rc;
    if ((rc = rms(e.x, Ly.post_norm, e.norm))) return rc;
    if ((rc = gemv(Ly.gu, e.norm, e.h, I, H))) return rc;
    if ((rc = gemv(Ly.gu + uint64_t{I} * H, e.norm, e.up, I, H))) return rc;
    if ((rc = L("QwenSiluMultiply", I / 32, {{8, &e.h}, {8, &e.up}, {4, &I}}))) return rc;
    if ((rc = gemv(Ly.down, e.h, e.tmp, H, I))) return rc;
    if ((rc = L("QwenAdd", H / 32, {{8, &e.x}, {8, &e.tmp}, {4, &H}}))) return rc;
  }
  if ((rc = rms(e.x, e.final_norm, e.norm))) return rc;
  if ((rc = gemv(e.lm_head, e.norm, e.logits, V, H))) return rc;
  if ((rc = L("QwenArgmax", 1, {{8, &e.logits}, {8, &e.ref_token}, {4, &V}}))) return rc;
  return xpu_rt_copy_from_device(rt, next, e.ref_token, 4);
}

int init_engine(xpu_qwen3 &e, xpu_runtime *rt, const xpu_qwen3_config &cfg, uint32_t max_seq) {
  int rc = validate_config(cfg);
  if (rc) return rc;
  if (max_seq == 0 || max_seq > kMaxContext)
    return set_error(XPU_ERR_INVALID, "max_seq must be in [1, 40960] (qwen3/main.cpp:69-70)");
  e.c = cfg;
  e.max_seq = max_seq;
  if (!rt) {
    if ((rc = xpu_rt_create(nullptr, -1, &e.rt))) return rc;
    e.owns_rt = true;
  } else {
    e.rt = rt;
  }
  plan_arena(e, nullptr);
  if ((rc = allocate_buffers(e))) return rc;
  plan_arena(e, e.arena);
  if ((rc = setup_launches(e))) return rc;
  return setup_prefill(e);
}

// ---------------------------------------------------------------- checkpoint

std::string read_text(const std::string &path, uint64_t limit = 1ull << 26) {
  std::ifstream f(path, std::ios::binary | std::ios::ate);
  if (!f) throw std::runtime_error("cannot open " + path);
  const auto n = f.tellg();
  if (n < 0 || static_cast<uint64_t>(n) > limit) throw std::runtime_error("invalid or too large file: " + path);
  std::string s(static_cast<size_t>(n), '\0');
  f.seekg(0);
  if (!f.read(s.data(), n)) throw std::runtime_error("cannot read " + path);
  return s;
}

// config.json (qwen3/model.cpp:376-410, generalised to the Qwen3 family)
xpu_qwen3_config parse_config(const std::string &model_dir) {
  using xpu::json::Node;
  using xpu::json::Type;
  const std::string path = model_dir + "/config.json";
  const xpu::json::Document doc(read_text(path), path);
  const Node root = doc.root();
  if (!root.is(Type::Object)) throw std::runtime_error(path + ": the document is not a JSON object");
  auto field = [&](const char *name) {
    const Node v = root.member(name);
    if (!v) throw std::runtime_error(path + ": missing field '" + name + "'");
    return v;
  };
  auto u32 = [&](const char *name) {
    uint64_t v = 0;
    if (!field(name).exact_u64(v) || v > 0xffffffffull)
      throw std::runtime_error(path + ": field '" + name + "' must be an unsigned 32-bit integer");
    return static_cast<uint32_t>(v);
  };
  auto str = [&](const char *name) {
    const Node v = field(name);
    if (!v.is(Type::String)) throw std::runtime_error(path + ": field '" + name + "' must be a string");
    return std::string(v.string());
  };
  xpu_qwen3_config c{};
  c.hidden = u32("hidden_size");
  c.intermediate = u32("intermediate_size");
  c.heads = u32("num_attention_heads");
  c.kv_heads = u32("num_key_value_heads");
  c.layers = u32("num_hidden_layers");
  c.vocab = u32("vocab_size");
  c.head_dim = root.member("head_dim") ? u32("head_dim") : (c.heads ? c.hidden / c.heads : 0);
  const Node eps = field("rms_norm_eps");
  if (!eps.is(Type::Number)) throw std::runtime_error(path + ": field 'rms_norm_eps' must be a number");
  c.rms_eps = static_cast<float>(eps.number());
  // transformers 5 nests rope_theta under rope_parameters
  Node theta = root.member("rope_theta");
  if (!theta) theta = root.member("rope_parameters").member("rope_theta");
  if (!theta.is(Type::Number)) throw std::runtime_error(path + ": missing numeric field 'rope_theta'");
  c.rope_theta = theta.number();
  c.tied = root.member("tie_word_embeddings").truth();
  if (str("model_type") != "qwen3") throw std::runtime_error("model_type must be qwen3");
  if (str("hidden_act") != "silu") throw std::runtime_error("hidden_act must be silu");
  Node dt = root.member("torch_dtype");
  if (!dt) dt = root.member("dtype");
  if (dt.string() != "bfloat16") throw std::runtime_error("checkpoint dtype must be bfloat16");
  if (const Node rs = root.member("rope_scaling"); rs && !rs.is(Type::Null))
    throw std::runtime_error("rope_scaling is not supported");
  return c;
}

struct StoredTensor {
  std::string file;
  uint64_t offset = 0, bytes = 0;
  std::vector<uint64_t> shape;
};

// Tensor directory of a checkpoint (qwen3/model.cpp:288-368,448-478): with
// an index, its weight_map names the shard of every tensor, each shard's
// header must list exactly the tensors mapped to it, and metadata.total_size
// must equal the payload bytes; without one, model.safetensors alone. Every
// tensor is BF16, its byte range lies inside its shard's payload (checked
// without overflow) and no two ranges of a shard overlap.
std::map<std::string, StoredTensor> read_safetensors(const std::string &dir) {
  using xpu::json::Node;
  using xpu::json::Type;
  std::map<std::string, std::set<std::string>> shards;  // shard -> tensors the index maps to it
  bool indexed = false;
  uint64_t total_size = 0;
  const std::string index_path = dir + "/model.safetensors.index.json";
  if (std::ifstream(index_path)) {
    indexed = true;
    const xpu::json::Document index(read_text(index_path), index_path);
    const Node map = index.root().member("weight_map");
    if (!map.is(Type::Object)) throw std::runtime_error(index_path + ": weight_map must be an object");
    map.each_member([&](std::string_view name, Node shard) {
      const std::string_view file = shard.string();
      if (!shard.is(Type::String) || file.empty() || file.find('/') != std::string_view::npos)
        throw std::runtime_error("invalid shard name for tensor " + std::string(name));
      for (const auto &other : shards)
        if (other.second.count(std::string(name))) throw std::runtime_error("tensor listed twice: " + std::string(name));
      shards[std::string(file)].insert(std::string(name));
    });
    if (!index.root().member("metadata").member("total_size").exact_u64(total_size))
      throw std::runtime_error(index_path + ": metadata.total_size must be an unsigned integer");
  } else {
    shards["model.safetensors"];
  }
  std::map<std::string, StoredTensor> out;
  uint64_t payload = 0;
  for (const auto &[name, mapped] : shards) {
    const std::string path = dir + "/" + name;
    std::ifstream f(path, std::ios::binary | std::ios::ate);
    if (!f) throw std::runtime_error("cannot open checkpoint shard " + path);
    const uint64_t size = static_cast<uint64_t>(f.tellg());
    f.seekg(0);
    unsigned char lenb[8];
    if (size < 8 || !f.read(reinterpret_cast<char *>(lenb), 8)) throw std::runtime_error("truncated " + path);
    uint64_t hlen = 0;
    for (int i = 0; i < 8; ++i) hlen |= uint64_t{lenb[i]} << (8 * i);
    if (hlen == 0 || hlen > (1ull << 30) || hlen > size - 8)
      throw std::runtime_error("invalid safetensors header length in " + path);
    std::string header(hlen, '\0');
    if (!f.read(header.data(), static_cast<std::streamsize>(hlen))) throw std::runtime_error("truncated " + path);
    const xpu::json::Document doc(header, path + " header");
    if (!doc.root().is(Type::Object)) throw std::runtime_error(path + ": header is not a JSON object");
    const uint64_t data_start = 8 + hlen, data_bytes = size - data_start;
    std::vector<std::pair<std::pair<uint64_t, uint64_t>, std::string>> ranges;
    size_t listed = 0;
    doc.root().each_member([&](std::string_view key, Node entry) {
      const std::string tname(key);
      if (tname == "__metadata__") return;
      if (indexed && !mapped.count(tname))
        throw std::runtime_error("shard " + name + " holds a tensor the index does not map to it: " + tname);
      ++listed;
      if (entry.member("dtype").string() != "BF16")
        throw std::runtime_error("tensor " + tname + " is not BF16 (qwen3/model.cpp:348-350)");
      StoredTensor t;
      t.file = path;
      uint64_t elems = 1;
      entry.member("shape").each_element([&](Node d) {
        uint64_t v = 0;
        if (!d.exact_u64(v) || v == 0 || elems > UINT64_MAX / 2 / v)
          throw std::runtime_error("invalid shape for tensor " + tname);
        t.shape.push_back(v);
        elems *= v;
      });
      const Node offs = entry.member("data_offsets");
      uint64_t b = 0, e = 0;
      if (offs.size() != 2 || !offs.element(0).exact_u64(b) || !offs.element(1).exact_u64(e) || e < b)
        throw std::runtime_error("invalid data offsets for tensor " + tname);
      if (e > data_bytes) throw std::runtime_error("tensor extends beyond shard: " + tname);
      t.offset = data_start + b;
      t.bytes = e - b;
      if (elems * 2 != t.bytes) throw std::runtime_error("byte size does not match BF16 shape for " + tname);
      payload += t.bytes;
      ranges.push_back({{b, e}, tname});
      if (!out.emplace(tname, std::move(t)).second) throw std::runtime_error("tensor listed twice: " + tname);
    });
    if (indexed && listed != mapped.size())
      for (const std::string &t : mapped)
        if (!out.count(t)) throw std::runtime_error("index names tensor absent from shard " + name + ": " + t);
    std::sort(ranges.begin(), ranges.end());
    for (size_t i = 1; i < ranges.size(); ++i)
      if (ranges[i].first.first < ranges[i - 1].first.second)
        throw std::runtime_error("overlapping safetensors payloads: " + ranges[i - 1].second + " and " +
                                 ranges[i].second);
  }
  if (indexed && payload != total_size)
    throw std::runtime_error("safetensors index total_size does not match tensor payloads");
  return out;
}

// The tensors a checkpoint of shape c must hold, with their engine kind and
// layer, each checked for presence and shape against the directory (tied
// checkpoints may also carry lm_head.weight, which is then ignored);
// qwen3/model.cpp:412-446 for the 8B shape, generalised.
using WantedTensor = std::pair<std::string, std::pair<int, uint32_t>>;
std::vector<WantedTensor> plan_checkpoint(const xpu_qwen3_config &c,
                                          const std::map<std::string, StoredTensor> &tensors) {
  const char *suffix[] = {"self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
                          "self_attn.o_proj.weight", "self_attn.q_norm.weight", "self_attn.k_norm.weight",
                          "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight",
                          "input_layernorm.weight", "post_attention_layernorm.weight"};
  auto shape_of = [&](int kind) -> std::vector<uint64_t> {
    const uint64_t H = c.hidden, qd = uint64_t{c.heads} * c.head_dim, kvd = uint64_t{c.kv_heads} * c.head_dim,
                   I = c.intermediate;
    switch (kind) {
      case XPU_W_Q: return {qd, H};
      case XPU_W_K: case XPU_W_V: return {kvd, H};
      case XPU_W_O: return {H, qd};
      case XPU_W_QNORM: case XPU_W_KNORM: return {c.head_dim};
      case XPU_W_GATE: case XPU_W_UP: return {I, H};
      case XPU_W_DOWN: return {H, I};
      case XPU_W_EMBED: case kLmHead: return {c.vocab, H};
      default: return {H};
    }
  };
  std::vector<WantedTensor> wanted;
  for (uint32_t l = 0; l < c.layers; ++l)
    for (int k = 0; k <= XPU_W_POSTNORM; ++k)
      wanted.push_back({"model.layers." + std::to_string(l) + "." + suffix[k], {k, l}});
  wanted.push_back({"model.embed_tokens.weight", {XPU_W_EMBED, 0}});
  wanted.push_back({"model.norm.weight", {XPU_W_FINALNORM, 0}});
  if (!c.tied) wanted.push_back({"lm_head.weight", {kLmHead, 0}});
  std::set<std::string> expected;
  for (auto &w : wanted) expected.insert(w.first);
  for (const auto &t : tensors)
    if (!expected.count(t.first) && !(c.tied && t.first == "lm_head.weight"))
      throw std::runtime_error("unexpected tensor in checkpoint: " + t.first);
  for (auto &w : wanted) {
    auto it = tensors.find(w.first);
    if (it == tensors.end()) throw std::runtime_error("checkpoint is missing tensor: " + w.first);
    if (it->second.shape != shape_of(w.second.first)) throw std::runtime_error("wrong shape for tensor " + w.first);
  }
  return wanted;
}

int load_checkpoint(xpu_qwen3 &e, const std::string &dir) {
  const auto tensors = read_safetensors(dir);
  const std::vector<WantedTensor> wanted = plan_checkpoint(e.c, tensors);
  std::vector<char> chunk(64u << 20);  // main.cpp:266: 64 MiB staging chunks
  for (auto &w : wanted) {
    auto it = tensors.find(w.first);
    std::ifstream f(it->second.file, std::ios::binary);
    f.seekg(static_cast<std::streamoff>(it->second.offset));
    uint8_t *dst = reinterpret_cast<uint8_t *>(tensor_location(e, w.second.first, w.second.second));
    uint64_t left = it->second.bytes;
    while (left) {
      const size_t n = static_cast<size_t>(std::min<uint64_t>(left, chunk.size()));
      if (!f.read(chunk.data(), static_cast<std::streamsize>(n)))
        return set_error(XPU_ERR_INVALID, "short read while streaming tensor " + w.first);
      const int rc = xpu_rt_copy_to_device(e.rt, dst, chunk.data(), n);
      if (rc) return rc;
      dst += n;
      left -= n;
    }
  }
  return XPU_OK;
}

}  // namespace

// ---------------------------------------------------------------- C ABI

extern "C" int xpu_qwen3_preset(const char *name, xpu_qwen3_config *out) {
  if (!name || !out) return set_error(XPU_ERR_INVALID, "null argument");
  const std::string n(name);
  xpu_qwen3_config c{};
  c.head_dim = 128;
  c.rms_eps = 1e-6f;
  c.rope_theta = 1e6;
  c.tied = 1;
  if (n == "qwen3-0.6b") { c.hidden = 1024; c.intermediate = 3072; c.layers = 28; c.heads = 16; c.kv_heads = 8; c.vocab = 151936; }
  else if (n == "qwen3-8b") { c.hidden = 4096; c.intermediate = 12288; c.layers = 36; c.heads = 32; c.kv_heads = 8; c.vocab = 151936; c.tied = 0; }
  else if (n == "tiny") { c.hidden = 256; c.intermediate = 512; c.layers = 2; c.heads = 4; c.kv_heads = 2; c.vocab = 1000; }
  else if (n == "small") { c.hidden = 1024; c.intermediate = 3072; c.layers = 2; c.heads = 16; c.kv_heads = 8; c.vocab = 4096; }
  else return set_error(XPU_ERR_INVALID, "unknown Qwen3 preset: " + n);
  *out = c;
  return XPU_OK;
}

extern "C" int xpu_qwen3_fill_tensor(const xpu_qwen3_config *cfg, uint64_t seed, float gain_std, int kind,
                                     uint32_t layer, uint16_t *out, uint64_t count) {
  if (!cfg || !out) return set_error(XPU_ERR_INVALID, "null argument");
  if (kind < 0 || kind >= static_cast<int>(kTensorKinds)) return set_error(XPU_ERR_INVALID, "bad tensor kind");
  if (count != tensor_elems(*cfg, kind)) return set_error(XPU_ERR_INVALID, "count does not match the tensor");
  fill_tensor(*cfg, seed, gain_std, kind, layer, out);
  return XPU_OK;
}

extern "C" int xpu_qwen3_rope_tables(uint16_t *cos_t, uint16_t *sin_t, uint32_t max_seq, uint32_t head_dim,
                                     double theta) {
  if (!cos_t || !sin_t || head_dim < 2 || head_dim % 2) return set_error(XPU_ERR_INVALID, "invalid RoPE table");
  // transformers Qwen3RotaryEmbedding: inv_freq = 1 / theta^(2i/d) in FP32,
  // angle = fp32(position * inv_freq), cos/sin of the FP32 angle; entry d
  // uses frequency d % (d/2) (qwen3/main.cpp:303-313 computes in double)
  const uint32_t half = head_dim / 2;
  std::vector<float> inv(half);
  for (uint32_t i = 0; i < half; ++i) {
    const float expo = static_cast<float>(2 * i) / static_cast<float>(head_dim);
    inv[i] = 1.0f / static_cast<float>(std::pow(static_cast<double>(static_cast<float>(theta)),
                                                static_cast<double>(expo)));
  }
  for (uint32_t p = 0; p < max_seq; ++p)
    for (uint32_t d = 0; d < head_dim; ++d) {
      const float angle = static_cast<float>(p) * inv[d % half];
      cos_t[uint64_t{p} * head_dim + d] = xpu::f32_to_bf16(static_cast<float>(std::cos(static_cast<double>(angle))));
      sin_t[uint64_t{p} * head_dim + d] = xpu::f32_to_bf16(static_cast<float>(std::sin(static_cast<double>(angle))));
    }
  return XPU_OK;
}

extern "C" int xpu_synth_tokens(uint32_t *out, uint64_t n, uint64_t seed, uint32_t vocab) {
  if (!out || !vocab) return set_error(XPU_ERR_INVALID, "invalid token request");
  for (uint64_t i = 0; i < n; ++i)
    out[i] = static_cast<uint32_t>(((xpu::counter_hash(seed, i) >> 32) * uint64_t{vocab}) >> 32);
  return XPU_OK;
}

extern "C" int xpu_qwen3_create(xpu_runtime *rt, const xpu_qwen3_config *cfg, uint32_t max_seq, uint64_t seed,
                                float gain_std, xpu_qwen3 **out) {
  if (!cfg || !out) return set_error(XPU_ERR_INVALID, "null argument");
  *out = nullptr;
  auto e = std::make_unique<xpu_qwen3>();
  int rc = init_engine(*e, rt, *cfg, max_seq);
  if (rc) return rc;
  // synthetic weights, generated on the host per logical tensor and placed
  // into the fused layout
  std::vector<uint16_t> host;
  auto upload = [&](int kind, uint32_t layer) {
    host.resize(tensor_elems(e->c, kind));
    fill_tensor(e->c, seed, gain_std, kind, layer, host.data());
    return xpu_rt_copy_to_device(e->rt, tensor_location(*e, kind, layer), host.data(), host.size() * 2);
  };
  for (uint32_t l = 0; l < e->c.layers; ++l)
    for (int kind = 0; kind <= XPU_W_POSTNORM; ++kind)
      if ((rc = upload(kind, l))) return rc;
  if ((rc = upload(XPU_W_EMBED, 0)) || (rc = upload(XPU_W_FINALNORM, 0))) return rc;
  if (!e->c.tied && (rc = upload(kLmHead, 0))) return rc;
  *out = e.release();
  return XPU_OK;
}

extern "C" int xpu_qwen3_read_config(const char *model_dir, xpu_qwen3_config *out) {
  if (!model_dir || !out) return set_error(XPU_ERR_INVALID, "null argument");
  try {
    const xpu_qwen3_config c = parse_config(model_dir);
    const int rc = validate_config(c);
    if (rc) return rc;
    *out = c;
    return XPU_OK;
  } catch (const std::exception &ex) {
    return set_error(XPU_ERR_INVALID, ex.what());
  }
}

extern "C" int xpu_qwen3_validate_checkpoint(const char *model_dir, xpu_qwen3_config *out) {
  if (!model_dir) return set_error(XPU_ERR_INVALID, "null argument");
  xpu_qwen3_config c{};
  int rc = xpu_qwen3_read_config(model_dir, &c);
  if (rc) return rc;
  try {
    plan_checkpoint(c, read_safetensors(model_dir));
  } catch (const std::exception &ex) {
    return set_error(XPU_ERR_INVALID, ex.what());
  }
  if (out) *out = c;
  return XPU_OK;
}

extern "C" int xpu_qwen3_create_from_checkpoint(xpu_runtime *rt, const char *model_dir, uint32_t max_seq,
                                                xpu_qwen3 **out) {
  if (!model_dir || !out) return set_error(XPU_ERR_INVALID, "null argument");
  *out = nullptr;
  xpu_qwen3_config c{};
  int rc = xpu_qwen3_read_config(model_dir, &c);
  if (rc) return rc;
  auto e = std::make_unique<xpu_qwen3>();
  if ((rc = init_engine(*e, rt, c, max_seq))) return rc;
  try {
    if ((rc = load_checkpoint(*e, model_dir))) return rc;
  } catch (const std::exception &ex) {
    return set_error(XPU_ERR_INVALID, ex.what());
  }
  *out = e.release();
  return XPU_OK;
}

extern "C" void xpu_qwen3_destroy(xpu_qwen3 *eng) { delete eng; }

extern "C" int xpu_qwen3_get_config(const xpu_qwen3 *eng, xpu_qwen3_config *out) {
  if (!eng || !out) return set_error(XPU_ERR_INVALID, "null argument");
  *out = eng->c;
  return XPU_OK;
}

extern "C" int xpu_qwen3_set_mode(xpu_qwen3 *eng, int mode) {
  if (!eng) return set_error(XPU_ERR_INVALID, "null engine");
  if (mode != XPU_QWEN3_GRAPH && mode != XPU_QWEN3_EAGER && mode != XPU_QWEN3_REFERENCE)
    return set_error(XPU_ERR_INVALID, "unknown Qwen3 mode");
  eng->mode = mode;
  return XPU_OK;
}

extern "C" int xpu_qwen3_set_prefill(xpu_qwen3 *eng, int mode) {
  if (!eng) return set_error(XPU_ERR_INVALID, "null engine");
  if (mode < 0 || mode > 2)
    return set_error(XPU_ERR_INVALID, "prefill mode must be 0 (stepwise), 1 (batched) or 2 (gemm)");
  if (mode == 1 && !eng->pf_ok)
    return set_error(XPU_ERR_INVALID, "batched prefill has no kernels for this model shape");
  if (mode == 2 && !eng->pf_gemm_ok)
    return set_error(XPU_ERR_INVALID, "gemm prefill has no kernels for this model shape");
  if (mode != 0) {
    const int rc = size_prompt_buffers(*eng, mode == 2);
    if (rc) return rc;
  }
  eng->batched_prefill = mode != 0;
  eng->gemm_prefill = mode == 2;
  return XPU_OK;
}

extern "C" int xpu_qwen3_set_attention_split(xpu_qwen3 *eng, uint32_t min_context) {
  if (!eng) return set_error(XPU_ERR_INVALID, "null engine");
  if (min_context && !eng->split_ok)
    return set_error(XPU_ERR_INVALID, "split attention has no kernels for this engine");
  eng->split_from = min_context;
  return XPU_OK;
}

namespace {

// The reference-mode kernels keep the caches position-major, the fused ones
// chunk-major: a step reads positions 0..position-1 from the caches, so it
// needs them written in its own mode's layout. Position 0 starts a new
// sequence in the current layout.
int claim_kv_layout(xpu_qwen3 &e, uint32_t position) {
  const int layout = e.mode == XPU_QWEN3_REFERENCE ? 1 : 0;
  if (position == 0) {
    e.kv_layout = layout;
    return XPU_OK;
  }
  if (e.kv_layout != -1 && e.kv_layout != layout)
    return set_error(XPU_ERR_INVALID,
                     "the KV cache holds this sequence in the other mode's layout (reference mode is "
                     "position-major, graph and eager modes chunk-major): after switching between them, "
                     "decode from position 0");
  return XPU_OK;
}

}  // namespace

extern "C" int xpu_qwen3_decode(xpu_qwen3 *eng, uint32_t token, uint32_t position, uint32_t *next) {
  if (!eng || !next) return set_error(XPU_ERR_INVALID, "null argument");
  if (token >= eng->c.vocab) return set_error(XPU_ERR_INVALID, "input token ID is outside the vocabulary");
  if (position >= eng->max_seq) return set_error(XPU_ERR_INVALID, "position exceeds --max-seq-len");
  int rc;
  if ((rc = claim_kv_layout(*eng, position))) return rc;
  uint32_t result = 0;
  if (eng->mode == XPU_QWEN3_REFERENCE) {
    if ((rc = reference_step(*eng, token, position, &result))) return rc;
  } else {
    const uint32_t st[4] = {position, token, 0, 0};
    if ((rc = xpu_rt_copy_to_device(eng->rt, eng->state, st, sizeof(st)))) return rc;
    if ((rc = set_rope_row(*eng, position))) return rc;
    if ((rc = run_fused_step(*eng, position))) return rc;
    uint32_t back[4];
    if ((rc = xpu_rt_copy_from_device(eng->rt, back, eng->state, sizeof(back)))) return rc;
    result = back[2];
  }
  if (result == 0xffffffffu)
    return set_error(XPU_ERR_VERIFY, "model produced a NaN or infinity in vocabulary logits");
  *next = result;
  return XPU_OK;
}

extern "C" int xpu_qwen3_logits(xpu_qwen3 *eng, uint16_t *out, uint64_t count) {
  if (!eng || !out || count > eng->c.vocab) return set_error(XPU_ERR_INVALID, "invalid logits request");
  return xpu_rt_copy_from_device(eng->rt, out, eng->logits, count * 2);
}

extern "C" int xpu_qwen3_hidden(xpu_qwen3 *eng, uint16_t *out, uint64_t count) {
  if (!eng || !out || count > eng->c.hidden) return set_error(XPU_ERR_INVALID, "invalid hidden request");
  return xpu_rt_copy_from_device(eng->rt, out, eng->x, count * 2);
}

extern "C" int xpu_qwen3_generate(xpu_qwen3 *eng, const uint32_t *prompt, uint32_t n_prompt, uint32_t max_new,
                                  int stop_on_eos, uint32_t *out, uint32_t *n_out, double *prompt_ms,
                                  double *decode_ms) {
  if (!eng || !prompt || !n_out || (max_new && !out)) return set_error(XPU_ERR_INVALID, "null argument");
  *n_out = 0;
  // main.cpp:90-100
  if (n_prompt == 0) return set_error(XPU_ERR_INVALID, "at least one input token ID is required");
  if (n_prompt > eng->max_seq || max_new > eng->max_seq - n_prompt)
    return set_error(XPU_ERR_INVALID, "prompt plus requested generation exceeds --max-seq-len");
  for (uint32_t i = 0; i < n_prompt; ++i)
    if (prompt[i] >= eng->c.vocab) return set_error(XPU_ERR_INVALID, "input token ID is outside the vocabulary");
  const uint32_t steps = n_prompt + std::max(max_new, 1u) - 1;
  int rc;
  if ((rc = claim_kv_layout(*eng, 0))) return rc;
  double p_ms = 0, d_ms = 0;
  std::vector<uint32_t> gen(std::max(max_new, 1u));
  if (eng->mode == XPU_QWEN3_REFERENCE) {
    auto t0 = std::chrono::steady_clock::now();
    uint32_t next = 0;
    for (uint32_t p = 0; p < n_prompt; ++p)
      if ((rc = xpu_qwen3_decode(eng, prompt[p], p, &next))) return rc;
    auto t1 = std::chrono::steady_clock::now();
    uint32_t produced = 0;
    for (uint32_t i = 0; i < max_new; ++i) {
      gen[produced++] = next;
      if (stop_on_eos && (next == kEos || next == kEndOfTurn)) break;
      if (i + 1 != max_new && (rc = xpu_qwen3_decode(eng, next, n_prompt + i, &next))) return rc;
    }
    auto t2 = std::chrono::steady_clock::now();
    p_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
    d_ms = std::chrono::duration<double, std::milli>(t2 - t1).count();
    std::copy(gen.begin(), gen.begin() + produced, out);
    *n_out = produced;
  } else {
    if ((rc = xpu_rt_copy_to_device(eng->rt, eng->prompt, prompt, n_prompt * 4ull))) return rc;
    // batched prefill of every prompt position, the last one finished by
    // the decode step's tail kernels (they yield the first new token); a
    // one-id prompt runs as a decode step
    const bool whole = eng->batched_prefill && n_prompt >= 2;
    const uint32_t first = eng->batched_prefill ? n_prompt - 1 : 0;
    const uint32_t st[4] = {first, prompt[first], 0, n_prompt};
    if ((rc = xpu_rt_copy_to_device(eng->rt, eng->state, st, sizeof(st)))) return rc;
    if ((rc = set_rope_row(*eng, first))) return rc;
    void *ev[3] = {nullptr, nullptr, nullptr};
    for (auto &v : ev)
      if ((rc = xpu_rt_event_create(eng->rt, &v))) return rc;
    rc = xpu_rt_event_record(eng->rt, ev[0]);
    if (!rc && whole) rc = run_prefill(*eng, n_prompt, true);
    if (!rc && whole) rc = xpu_rt_event_record(eng->rt, ev[1]);
    for (uint32_t s = whole ? n_prompt : first; !rc && s < steps; ++s) {
      rc = run_fused_step(*eng, s);
      if (!rc && s + 1 == n_prompt) rc = xpu_rt_event_record(eng->rt, ev[1]);
    }
    if (!rc) rc = xpu_rt_event_record(eng->rt, ev[2]);
    float a = 0, b = 0;
    if (!rc) rc = xpu_rt_event_elapsed_ms(ev[0], ev[1], &a);
    if (!rc) rc = xpu_rt_event_elapsed_ms(ev[1], ev[2], &b);
    for (auto &v : ev) xpu_rt_event_destroy(v);
    if (rc) return rc;
    p_ms = a;
    d_ms = b;
    if (max_new && (rc = xpu_rt_copy_from_device(eng->rt, gen.data(), eng->gen, max_new * 4ull))) return rc;
    uint32_t produced = 0;
    for (uint32_t i = 0; i < max_new; ++i) {
      if (gen[i] == 0xffffffffu)
        return set_error(XPU_ERR_VERIFY, "model produced a NaN or infinity in vocabulary logits");
      out[produced++] = gen[i];
      if (stop_on_eos && (gen[i] == kEos || gen[i] == kEndOfTurn)) break;
    }
    *n_out = produced;
  }
  if (prompt_ms) *prompt_ms = p_ms;
  if (decode_ms) *decode_ms = d_ms;
  return XPU_OK;
}

// ---------------------------------------------------------------- run_qwen3

namespace {

struct QwenOptions {
  std::string model_dir, input_ids, synthetic;
  uint32_t max_new_tokens = 0, max_sequence = kMaxContext;
  bool has_max_new_tokens = false, stop_on_eos = true;
  uint64_t seed = 0;
  float gain_std = 0.0f;
  int mode = XPU_QWEN3_GRAPH;
  int prefill = -1;  // -1: the engine's default
};

[[noreturn]] void qwen_usage_error(const std::string &message) {
  throw std::invalid_argument(message +
                              "\nUsage: qwen3_hip --model-dir DIR | --synthetic PRESET --input-ids FILE|- "
                              "--max-new-tokens N [--max-seq-len N]");
}

uint32_t parse_u32(const std::string &text, const std::string &option, bool allow_zero) {
  size_t used = 0;
  unsigned long long v = 0;
  try {
    v = std::stoull(text, &used);
  } catch (...) {
    qwen_usage_error("invalid value for " + option + ": " + text);
  }
  if (used != text.size() || v > 0xffffffffull || (!allow_zero && v == 0))
    qwen_usage_error("invalid value for " + option + ": " + text);
  return static_cast<uint32_t>(v);
}

// main.cpp:43-72
QwenOptions parse_qwen(int argc, char **argv) {
  QwenOptions o;
  for (int i = 1; i < argc; ++i) {
    const std::string opt = argv[i];
    if (opt == "-h" || opt == "--help") {
      std::cout << "Usage: " << argv[0]
                << " --model-dir DIR | --synthetic qwen3-0.6b|qwen3-8b|tiny|small [--seed N] [--gain-std X]\n"
                   "       --input-ids FILE|- --max-new-tokens N [--max-seq-len N]\n"
                   "       [--mode graph|eager|reference] [--prefill batched|gemm|stepwise] [--no-eos-stop]\n";
      std::exit(0);
    }
    if (opt == "--no-eos-stop") { o.stop_on_eos = false; continue; }
    if (i + 1 == argc) qwen_usage_error("missing value for " + opt);
    const std::string v = argv[++i];
    if (opt == "--model-dir") o.model_dir = v;
    else if (opt == "--synthetic") o.synthetic = v;
    else if (opt == "--input-ids") o.input_ids = v;
    else if (opt == "--max-new-tokens") { o.max_new_tokens = parse_u32(v, opt, true); o.has_max_new_tokens = true; }
    else if (opt == "--max-seq-len") o.max_sequence = parse_u32(v, opt, false);
    else if (opt == "--seed") o.seed = std::stoull(v);
    else if (opt == "--gain-std") o.gain_std = std::stof(v);
    else if (opt == "--mode") {
      if (v == "graph") o.mode = XPU_QWEN3_GRAPH;
      else if (v == "eager") o.mode = XPU_QWEN3_EAGER;
      else if (v == "reference") o.mode = XPU_QWEN3_REFERENCE;
      else qwen_usage_error("--mode must be graph, eager or reference");
    } else if (opt == "--prefill") {
      if (v == "batched") o.prefill = 1;
      else if (v == "stepwise") o.prefill = 0;
      else if (v == "gemm") o.prefill = 2;
      else qwen_usage_error("--prefill must be batched, gemm or stepwise");
    } else {
      qwen_usage_error("unknown option: " + opt);
    }
  }
  if (o.model_dir.empty() == o.synthetic.empty()) qwen_usage_error("exactly one of --model-dir and --synthetic is required");
  if (o.input_ids.empty()) qwen_usage_error("--input-ids is required");
  if (!o.has_max_new_tokens) qwen_usage_error("--max-new-tokens is required");
  if (o.max_sequence > kMaxContext) qwen_usage_error("--max-seq-len cannot exceed 40960");
  return o;
}

// main.cpp:74-102
std::vector<uint32_t> read_ids(const QwenOptions &o, uint32_t vocab) {
  std::ifstream file;
  std::istream *in = &std::cin;
  if (o.input_ids != "-") {
    file.open(o.input_ids);
    if (!file) throw std::runtime_error("cannot open input token file: " + o.input_ids);
    in = &file;
  }
  std::vector<uint32_t> ids;
  std::string tok;
  while (*in >> tok) {
    size_t used = 0;
    unsigned long long id = 0;
    try {
      id = std::stoull(tok, &used);
    } catch (...) {
      throw std::runtime_error("invalid input token ID: " + tok);
    }
    if (used != tok.size() || id >= vocab)
      throw std::runtime_error("input token ID is outside [0, " + std::to_string(vocab - 1) + "]: " + tok);
    ids.push_back(static_cast<uint32_t>(id));
  }
  if (!in->eof()) throw std::runtime_error("failed while reading input token IDs");
  if (ids.empty()) throw std::runtime_error("at least one input token ID is required");
  if (ids.size() > o.max_sequence || o.max_new_tokens > o.max_sequence - ids.size())
    throw std::runtime_error("prompt plus requested generation exceeds --max-seq-len");
  return ids;
}

}  // namespace

extern "C" int run_qwen3(int argc, char **argv) {
  xpu_qwen3 *eng = nullptr;
  try {
    const QwenOptions o = parse_qwen(argc, argv);
    xpu_qwen3_config cfg{};
    if (!o.synthetic.empty()) {
      if (xpu_qwen3_preset(o.synthetic.c_str(), &cfg)) throw std::runtime_error(xpu_last_error());
    } else if (xpu_qwen3_read_config(o.model_dir.c_str(), &cfg)) {
      throw std::runtime_error(xpu_last_error());
    }
    const std::vector<uint32_t> prompt = read_ids(o, cfg.vocab);
    const auto t0 = std::chrono::steady_clock::now();
    const int rc = o.synthetic.empty()
                       ? xpu_qwen3_create_from_checkpoint(nullptr, o.model_dir.c_str(), o.max_sequence, &eng)
                       : xpu_qwen3_create(nullptr, &cfg, o.max_sequence, o.seed, o.gain_std, &eng);
    if (rc) throw std::runtime_error(xpu_last_error());
    const double load_s = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    if (xpu_qwen3_set_mode(eng, o.mode)) throw std::runtime_error(xpu_last_error());
    if (o.prefill >= 0 && xpu_qwen3_set_prefill(eng, o.prefill)) throw std::runtime_error(xpu_last_error());
    std::cerr << "qwen3_hip: " << eng->rt->name << " (" << eng->rt->arch << "), " << cfg.layers << " layers, hidden "
              << cfg.hidden << ", weights " << (eng->arena_bytes >> 20) << " MiB loaded in " << load_s << " s\n";
    std::vector<uint32_t> out(std::max(o.max_new_tokens, 1u));
    uint32_t n = 0;
    double pm = 0, dm = 0;
    if (xpu_qwen3_generate(eng, prompt.data(), static_cast<uint32_t>(prompt.size()), o.max_new_tokens,
                           o.stop_on_eos, out.data(), &n, &pm, &dm))
      throw std::runtime_error(xpu_last_error());
    std::cerr << "qwen3_hip: prompt " << prompt.size() << " tokens in " << pm << " ms ("
              << prompt.size() / (pm * 1e-3) << " tok/s); " << (n ? n - 1 : 0) << " decode steps in " << dm
              << " ms (" << (n > 1 ? (n - 1) / (dm * 1e-3) : 0.0) << " tok/s)\n";
    // main.cpp:353-358
    std::cout << "{\"generated_ids\":[";
    for (uint32_t i = 0; i < n; ++i) std::cout << (i ? "," : "") << out[i];
    std::cout << "]}\n";
    xpu_qwen3_destroy(eng);
    return 0;
  } catch (const std::exception &error) {
    xpu_qwen3_destroy(eng);
    std::cerr << "qwen3_hip: " << error.what() << '\n';
    return 1;
  }
}
