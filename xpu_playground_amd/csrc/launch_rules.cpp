// Work-item launch rules for the kernels launchable by entry-name fragment
// (xpu_rt_launch). The reference derives the group count from work items
// and a per-kernel local size (qwen3/level_zero_runtime.cpp:148-155, 248);
// here each rule maps the same work-item counts the reference engine passes
// (qwen3/main.cpp:162-220) to a gfx950 geometry.
#include "runtime_internal.hpp"

#include <algorithm>
#include <cstring>

namespace xpu {
namespace {

uint32_t div_up(uint64_t a, uint64_t b) { return static_cast<uint32_t>((a + b - 1) / b); }
uint32_t lds_for(uint32_t width) { return ((width + 511u) & ~511u) * 2u; }

// QwenEmbedding(table, out, token, hidden): work items = hidden (main.cpp:162)
int embedding_geometry(uint32_t items, const xpu_kernel_arg *, const xpu_runtime &, Geometry &g) {
  g = {div_up(items, 256), 256, 0};
  return XPU_OK;
}

// QwenRmsNorm(in, w, out, width, eps): one work item (main.cpp:248)
int rmsnorm_geometry(uint32_t items, const xpu_kernel_arg *args, const xpu_runtime &rt, Geometry &g) {
  const uint32_t width = arg_value<uint32_t>(args, 3);
  if (width == 0) return set_error(XPU_ERR_INVALID, "QwenRmsNorm: width must be positive");
  g = {items ? 1u : 0u, 256, lds_for(width)};
  if (g.shared > rt.max_shared) return set_error(XPU_ERR_INVALID, "QwenRmsNorm: width too large");
  return XPU_OK;
}

// QwenGemv(A, x, y, rows, cols): work items = rows (main.cpp:255)
int gemv_geometry(uint32_t items, const xpu_kernel_arg *args, const xpu_runtime &rt, Geometry &g) {
  const uint32_t cols = arg_value<uint32_t>(args, 4);
  if (cols == 0) return set_error(XPU_ERR_INVALID, "QwenGemv: columns must be positive");
  g.block = 256;
  g.shared = lds_for(cols);
  if (g.shared > rt.max_shared) return set_error(XPU_ERR_INVALID, "QwenGemv: columns too large");
  g.grid = std::min<uint32_t>(div_up(items, 8), rt.compute_units * 4);
  return XPU_OK;
}

// QwenQkvRopeCache(...): work items = query heads (main.cpp:183)
int qkv_rope_geometry(uint32_t items, const xpu_kernel_arg *args, const xpu_runtime &, Geometry &g) {
  const uint32_t heads = arg_value<uint32_t>(args, 11), kv = arg_value<uint32_t>(args, 12);
  if (heads == 0 || kv == 0 || heads % kv != 0 || items > heads)
    return set_error(XPU_ERR_INVALID, "QwenQkvRopeCache: invalid head counts");
  g = {items, 64, 0};
  return XPU_OK;
}

// QwenAttention(q, kc, vc, out, pos, heads, kv_heads): work items = heads (main.cpp:191)
int attention_geometry(uint32_t items, const xpu_kernel_arg *args, const xpu_runtime &, Geometry &g) {
  const uint32_t heads = arg_value<uint32_t>(args, 5), kv = arg_value<uint32_t>(args, 6);
  if (heads == 0 || kv == 0 || heads % kv != 0 || items > heads)
    return set_error(XPU_ERR_INVALID, "QwenAttention: invalid head counts");
  g = {items, 256, 0};
  return XPU_OK;
}

// QwenAdd / QwenSiluMultiply(a, b, width): work items = width / 32 (main.cpp:206,261)
int elementwise_geometry(uint32_t, const xpu_kernel_arg *args, const xpu_runtime &, Geometry &g) {
  const uint32_t width = arg_value<uint32_t>(args, 2);
  g = {div_up(width, 256), 256, 0};
  return XPU_OK;
}

// QwenArgmax(logits, token, width): one work item (main.cpp:218)
int argmax_geometry(uint32_t items, const xpu_kernel_arg *, const xpu_runtime &, Geometry &g) {
  g = {items ? 1u : 0u, 1024, 0};
  return XPU_OK;
}

const LaunchRule kRules[] = {
    {"QwenEmbedding", "ppuu", embedding_geometry},
    {"QwenRmsNorm", "pppuf", rmsnorm_geometry},
    {"QwenGemv", "pppuu", gemv_geometry},
    {"QwenQkvRopeCache", "pppppppppuuuu", qkv_rope_geometry},
    {"QwenAttention", "ppppuuu", attention_geometry},
    {"QwenAdd", "ppu", elementwise_geometry},
    {"QwenSiluMultiply", "ppu", elementwise_geometry},
    {"QwenArgmax", "ppu", argmax_geometry},
};

}  // namespace

const LaunchRule *find_rule(const std::string &kernel_name) {
  for (const LaunchRule &r : kRules)
    if (kernel_name == r.name) return &r;
  return nullptr;
}

}  // namespace xpu
