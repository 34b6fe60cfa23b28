// Synthetic-input kernels: the seeded U[-1,1) generator shared with the CPU
// oracle, and the reference's hash initialisation of the GEMV benchmark
// (gemv.cpp:91-103).
#include "device_common.hpp"

namespace xpu {

XPU_DEVICE uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

}  // namespace xpu

// dst[i] = encode(dtype, (2u - 2^24) / 2^24), u = top 24 bits of
// mix64(mixed_seed + (i + 1) * 0x9e3779b97f4a7c15); mixed_seed = mix64(seed).
extern "C" __global__ __launch_bounds__(256) void xpu_fill_uniform_u16(
    uint16_t *__restrict__ dst, uint64_t n, uint64_t mixed_seed, uint32_t dtype) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    const uint64_t h = xpu::mix64(mixed_seed + (i + 1) * 0x9e3779b97f4a7c15ull);
    const int32_t u = static_cast<int32_t>(h >> 40);
    const float v = static_cast<float>(2 * u - (1 << 24)) * 0x1p-24f;
    dst[i] = static_cast<uint16_t>(dtype ? xpu::f32_to_fp16(v) : xpu::f32_to_bf16(v));
  }
}

// gemv.cpp:91-103: matrix element at linear index id of the (m x ld) matrix
// from a 32-bit integer hash of id, vector element c from c * 747796405.
extern "C" __global__ __launch_bounds__(256) void xpu_fill_reference_gemv(
    uint16_t *__restrict__ matrix, uint16_t *__restrict__ vector, uint32_t m, uint32_t k,
    uint32_t ld, uint32_t dtype) {
  const uint64_t total = static_cast<uint64_t>(m) * ld;
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  for (uint64_t id = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; id < total;
       id += stride) {
    uint32_t bits = static_cast<uint32_t>(id);
    bits ^= bits >> 16;
    bits *= 0x7feb352du;
    bits ^= bits >> 15;
    bits *= 0x846ca68bu;
    bits ^= bits >> 16;
    const float v = 0.25f + static_cast<float>(bits & 255u) / 1024.0f;
    matrix[id] = static_cast<uint16_t>(dtype ? xpu::f32_to_fp16(v) : xpu::f32_to_bf16(v));
    if (id < k) {
      const uint32_t vb = static_cast<uint32_t>(id) * 747796405u;
      const float xv = 0.5f + static_cast<float>((vb >> 16) & 127u) / 512.0f;
      vector[id] = static_cast<uint16_t>(dtype ? xpu::f32_to_fp16(xv) : xpu::f32_to_bf16(xv));
    }
  }
}

// Plain streaming copy of n16 16-byte words, the known-traffic reference
// against which the HBM byte counters of the other kernels are scaled.
extern "C" __global__ __launch_bounds__(256) void xpu_stream_copy(const xpu::u32x4 *__restrict__ src,
                                                                 xpu::u32x4 *__restrict__ dst, uint64_t n16) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n16; i += stride)
    dst[i] = __builtin_nontemporal_load(src + i);
}
