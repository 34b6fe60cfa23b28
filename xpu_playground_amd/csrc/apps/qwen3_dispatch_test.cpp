// Dispatch test of the eight Qwen3 reference-named kernels through the C++
// runtime wrapper (HipRuntime): the same known-answer checks the reference
// runs against its Level Zero runtime (qwen3/tests/test_gpu_dispatch.cpp:43-209),
// at the Qwen3-8B head layout (32 query / 8 KV heads) and the 0.6B layout
// (16 / 8). Usage: qwen3_dispatch_test [code object path]
#include "xpu_runtime.hpp"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <iostream>
#include <limits>
#include <string>
#include <vector>

namespace {

using bf16 = std::uint16_t;
constexpr std::uint32_t kHeadDim = 128;
constexpr std::uint32_t kMaximumContext = 40960;
constexpr std::uint32_t kVocabulary = 151936;

struct Shape {
  const char *name;
  std::uint32_t hidden, intermediate, heads, kv_heads;
};

// Round to nearest even through the integer form (qwen3/model.cpp:497-502).
bf16 b(float value) {
  std::uint32_t bits;
  std::memcpy(&bits, &value, 4);
  return static_cast<bf16>((bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16);
}
float f(bf16 value) {
  const std::uint32_t bits = static_cast<std::uint32_t>(value) << 16;
  float out;
  std::memcpy(&out, &bits, 4);
  return out;
}

void expect(bool ok, const std::string &what) {
  if (!ok) throw std::runtime_error("check failed: " + what);
}

void close(float actual, float expected, const std::string &what, float atol = 0.03f, float rtol = 0.02f) {
  if (!std::isfinite(actual) || std::abs(actual - expected) > atol + rtol * std::abs(expected))
    throw std::runtime_error(what + ": actual " + std::to_string(actual) + " expected " +
                             std::to_string(expected));
}

template <typename T> T *device_vector(xpu::HipRuntime &rt, const std::vector<T> &host) {
  auto *d = static_cast<T *>(rt.allocate_device(host.size() * sizeof(T), 64));
  rt.copy_to_device(d, host.data(), host.size() * sizeof(T));
  return d;
}

template <typename T> std::vector<T> download(xpu::HipRuntime &rt, const T *d, std::size_t n) {
  std::vector<T> out(n);
  rt.copy_from_device(out.data(), d, n * sizeof(T));
  return out;
}

void embedding(xpu::HipRuntime &rt, const Shape &s) {
  // row 3 of a 4-row table: out = table[3 * hidden ...]
  std::vector<bf16> table(4 * s.hidden);
  for (std::uint32_t i = 0; i < table.size(); ++i) table[i] = b((int(i % 29) - 14) / 16.0f);
  auto *d_table = device_vector(rt, table);
  auto *out = static_cast<bf16 *>(rt.allocate_device(s.hidden * 2, 64));
  std::uint32_t token = 3, hidden = s.hidden;
  rt.launch("QwenEmbedding", s.hidden,
            {xpu::kernel_argument(d_table), xpu::kernel_argument(out), xpu::kernel_argument(token),
             xpu::kernel_argument(hidden)});
  const auto host = download(rt, out, s.hidden);
  expect(std::equal(host.begin(), host.end(), table.begin() + 3 * s.hidden), "QwenEmbedding row copy");
}

void rms_norm(xpu::HipRuntime &rt, const Shape &s) {
  for (std::uint32_t width : {128u, s.hidden}) {
    std::vector<bf16> input(width), weight(width, b(0.75f));
    float squares = 0;
    for (std::uint32_t i = 0; i < width; ++i) {
      input[i] = b((int(i % 31) - 15) / 32.0f);
      squares += f(input[i]) * f(input[i]);
    }
    auto *d_in = device_vector(rt, input);
    auto *d_w = device_vector(rt, weight);
    auto *out = static_cast<bf16 *>(rt.allocate_device(width * 2, 64));
    float epsilon = 1.0e-6f;
    rt.launch("QwenRmsNorm", 1,
              {xpu::kernel_argument(d_in), xpu::kernel_argument(d_w), xpu::kernel_argument(out),
               xpu::kernel_argument(width), xpu::kernel_argument(epsilon)});
    const auto host = download(rt, out, width);
    const float scale = 1.0f / std::sqrt(squares / width + epsilon);
    for (std::uint32_t i = 0; i < width; ++i)
      close(f(host[i]), f(input[i]) * f(weight[i]) * scale, "QwenRmsNorm");
  }
}

void gemv(xpu::HipRuntime &rt) {
  std::uint32_t rows = 32, columns = 32;
  std::vector<bf16> matrix(rows * columns), vec(columns);
  for (std::uint32_t k = 0; k < columns; ++k) vec[k] = b((int(k % 7) - 3) / 8.0f);
  for (std::uint32_t i = 0; i < matrix.size(); ++i) matrix[i] = b((int(i % 11) - 5) / 16.0f);
  auto *d_m = device_vector(rt, matrix);
  auto *d_v = device_vector(rt, vec);
  auto *out = static_cast<bf16 *>(rt.allocate_device(rows * 2, 64));
  rt.launch("QwenGemv", rows,
            {xpu::kernel_argument(d_m), xpu::kernel_argument(d_v), xpu::kernel_argument(out),
             xpu::kernel_argument(rows), xpu::kernel_argument(columns)});
  const auto host = download(rt, out, rows);
  for (std::uint32_t r = 0; r < rows; ++r) {
    float expected = 0;
    for (std::uint32_t k = 0; k < columns; ++k) expected += f(matrix[r * columns + k]) * f(vec[k]);
    close(f(host[r]), expected, "QwenGemv row " + std::to_string(r));
  }
}

void qkv_rope_cache_and_attention(xpu::HipRuntime &rt, const Shape &s) {
  std::vector<bf16> query(s.heads * kHeadDim), key(s.kv_heads * kHeadDim), value(key.size());
  std::vector<bf16> norm(kHeadDim, b(1.0f)), cosine(kHeadDim, b(1.0f)), sine(kHeadDim, b(0.0f));
  for (std::uint32_t i = 0; i < query.size(); ++i) query[i] = b((int(i % 17) - 8) / 16.0f);
  for (std::uint32_t i = 0; i < key.size(); ++i) {
    key[i] = b((int(i % 13) - 6) / 16.0f);
    value[i] = b((int(i % 19) - 9) / 16.0f);
  }
  auto *d_q = device_vector(rt, query);
  auto *d_k = device_vector(rt, key);
  auto *d_v = device_vector(rt, value);
  auto *d_norm = device_vector(rt, norm);
  auto *d_cos = device_vector(rt, cosine);
  auto *d_sin = device_vector(rt, sine);
  auto *kc = static_cast<bf16 *>(rt.allocate_device(key.size() * 2, 64));
  auto *vc = static_cast<bf16 *>(rt.allocate_device(value.size() * 2, 64));
  std::uint32_t position = 0, maximum = 1, heads = s.heads, kv_heads = s.kv_heads;
  rt.launch("QwenQkvRopeCache", s.heads,
            {xpu::kernel_argument(d_q), xpu::kernel_argument(d_k), xpu::kernel_argument(d_v),
             xpu::kernel_argument(d_norm), xpu::kernel_argument(d_norm), xpu::kernel_argument(d_cos),
             xpu::kernel_argument(d_sin), xpu::kernel_argument(kc), xpu::kernel_argument(vc),
             xpu::kernel_argument(position), xpu::kernel_argument(maximum), xpu::kernel_argument(heads),
             xpu::kernel_argument(kv_heads)});
  expect(download(rt, vc, value.size()) == value, "QwenQkvRopeCache value slot");
  auto *attn = static_cast<bf16 *>(rt.allocate_device(query.size() * 2, 64));
  rt.launch("QwenAttention", s.heads,
            {xpu::kernel_argument(d_q), xpu::kernel_argument(kc), xpu::kernel_argument(vc),
             xpu::kernel_argument(attn), xpu::kernel_argument(position), xpu::kernel_argument(heads),
             xpu::kernel_argument(kv_heads)});
  // one cached position: softmax weight 1, output = V of kv head h / group
  const auto host = download(rt, attn, query.size());
  const std::uint32_t group = s.heads / s.kv_heads;
  for (std::uint32_t h = 0; h < s.heads; ++h)
    for (std::uint32_t i = 0; i < kHeadDim; ++i)
      close(f(host[h * kHeadDim + i]), f(value[(h / group) * kHeadDim + i]), "QwenAttention pos 0");

  // the last production cache slot (position 40959)
  const std::uint64_t cache_elements = std::uint64_t(kMaximumContext) * s.kv_heads * kHeadDim;
  auto *last_k = static_cast<bf16 *>(rt.allocate_device(cache_elements * 2));
  auto *last_v = static_cast<bf16 *>(rt.allocate_device(cache_elements * 2));
  const std::uint64_t rope_elements = std::uint64_t(kMaximumContext) * kHeadDim;
  auto *full_cos = static_cast<bf16 *>(rt.allocate_device(rope_elements * 2));
  auto *full_sin = static_cast<bf16 *>(rt.allocate_device(rope_elements * 2));
  const std::uint64_t rope_offset = std::uint64_t(kMaximumContext - 1) * kHeadDim;
  rt.copy_to_device(full_cos + rope_offset, cosine.data(), cosine.size() * 2);
  rt.copy_to_device(full_sin + rope_offset, sine.data(), sine.size() * 2);
  position = kMaximumContext - 1;
  maximum = kMaximumContext;
  rt.launch("QwenQkvRopeCache", s.heads,
            {xpu::kernel_argument(d_q), xpu::kernel_argument(d_k), xpu::kernel_argument(d_v),
             xpu::kernel_argument(d_norm), xpu::kernel_argument(d_norm), xpu::kernel_argument(full_cos),
             xpu::kernel_argument(full_sin), xpu::kernel_argument(last_k), xpu::kernel_argument(last_v),
             xpu::kernel_argument(position), xpu::kernel_argument(maximum), xpu::kernel_argument(heads),
             xpu::kernel_argument(kv_heads)});
  expect(download(rt, last_v + (cache_elements - value.size()), value.size()) == value,
         "QwenQkvRopeCache final slot");
  for (void *p : {static_cast<void *>(last_k), static_cast<void *>(last_v), static_cast<void *>(full_cos),
                  static_cast<void *>(full_sin)})
    rt.free_device(p);
}

void elementwise_and_argmax(xpu::HipRuntime &rt, const Shape &s) {
  std::uint32_t width = s.intermediate;
  std::vector<bf16> left(width), right(width);
  for (std::uint32_t i = 0; i < width; ++i) {
    left[i] = b((int(i % 11) - 5) / 8.0f);
    right[i] = b((int(i % 7) - 3) / 8.0f);
  }
  auto *d_l = device_vector(rt, left);
  auto *d_r = device_vector(rt, right);
  rt.launch("QwenAdd", width / 32, {xpu::kernel_argument(d_l), xpu::kernel_argument(d_r), xpu::kernel_argument(width)});
  auto host = download(rt, d_l, width);
  for (std::uint32_t i = 0; i < width; ++i) close(f(host[i]), f(left[i]) + f(right[i]), "QwenAdd");
  rt.copy_to_device(d_l, left.data(), left.size() * 2);
  rt.launch("QwenSiluMultiply", width / 32,
            {xpu::kernel_argument(d_l), xpu::kernel_argument(d_r), xpu::kernel_argument(width)});
  host = download(rt, d_l, width);
  for (std::uint32_t i = 0; i < width; ++i) {
    const float g = f(left[i]);
    close(f(host[i]), g / (1.0f + std::exp(-g)) * f(right[i]), "QwenSiluMultiply");
  }

  width = kVocabulary;
  std::vector<bf16> logits(width, b(-1.0f));
  logits[17] = logits[42] = b(3.0f);
  auto *d_logits = device_vector(rt, logits);
  auto *d_token = static_cast<std::uint32_t *>(rt.allocate_device(4, 64));
  rt.launch("QwenArgmax", 1,
            {xpu::kernel_argument(d_logits), xpu::kernel_argument(d_token), xpu::kernel_argument(width)});
  expect(download(rt, d_token, 1)[0] == 17, "QwenArgmax first maximum");
  logits[3] = b(std::numeric_limits<float>::quiet_NaN());
  rt.copy_to_device(d_logits, logits.data(), logits.size() * 2);
  rt.launch("QwenArgmax", 1,
            {xpu::kernel_argument(d_logits), xpu::kernel_argument(d_token), xpu::kernel_argument(width)});
  expect(download(rt, d_token, 1)[0] == 0xffffffffu, "QwenArgmax NaN sentinel");
}

}  // namespace

int main(int argc, char **argv) {
  try {
    xpu::HipRuntime rt(argc == 2 ? argv[1] : "");
    rt.require_device_and_memory(512ull << 20);
    for (const Shape &s : {Shape{"qwen3-8b", 4096, 12288, 32, 8}, Shape{"qwen3-0.6b", 1024, 3072, 16, 8}}) {
      embedding(rt, s);
      rms_norm(rt, s);
      gemv(rt);
      qkv_rope_cache_and_attention(rt, s);
      elementwise_and_argmax(rt, s);
      std::cout << "shape " << s.name << ": ok\n";
    }
    std::cout << "Qwen3 gfx950 kernel dispatch: PASS on " << rt.device_name() << '\n';
  } catch (const std::exception &error) {
    std::cerr << "Qwen3 gfx950 dispatch test: " << error.what() << '\n';
    return 1;
  }
  return 0;
}
