// Peak-rate microbenchmarks for gfx950: the measured denominators of the
// HBM and MFMA rooflines (reference: peak_mem_2d_kernel.cpp:13-52 and
// peak_compute_dpas_kernel.cpp:10-68, which do the same for the Xe2 block
// loads and DPAS).
#include "device_common.hpp"

namespace xpu {
typedef __bf16 peak_bf16x8 __attribute__((ext_vector_type(8)));
typedef float peak_f32x16 __attribute__((ext_vector_type(16)));
}  // namespace xpu

// Every wavefront runs `rounds` batches of 8 independent
// v_mfma_f32_32x32x16_bf16 (8 accumulator chains, as the reference's eight
// DPAS chains, peak_compute_dpas_kernel.cpp:38-58) on operands of 0.5, so
// each MFMA adds 16 * 0.25 = 4 to every accumulator element. Thread t writes
// the sum of element 0 of its 8 accumulators (28 + 32 * rounds) to sink[t].
// The first wavefront of block 0 also records the shader clock (s_memtime)
// and the constant-rate clock (s_memrealtime) around its loop in clock[0..3].
extern "C" __global__ __launch_bounds__(256) void xpu_peak_mfma_bf16(
    const uint16_t *__restrict__ operand, float *__restrict__ sink, uint64_t *__restrict__ clock,
    uint32_t rounds) {
  const xpu::u32x4 raw = *reinterpret_cast<const xpu::u32x4 *>(operand);
  const xpu::peak_bf16x8 a = __builtin_bit_cast(xpu::peak_bf16x8, raw);
  xpu::peak_f32x16 c[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) c[i][v] = static_cast<float>(i);
  const bool timer = blockIdx.x == 0 && threadIdx.x < 64;
  uint64_t t0 = 0, r0 = 0;
  if (timer) {
    t0 = __builtin_amdgcn_s_memtime();
    r0 = __builtin_amdgcn_s_memrealtime();
  }
#pragma unroll 1
  for (uint32_t r = 0; r < rounds; ++r) {
#pragma unroll
    for (int i = 0; i < 8; ++i) c[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, a, c[i], 0, 0, 0);
  }
  if (timer) {
    const uint64_t t1 = __builtin_amdgcn_s_memtime();
    const uint64_t r1 = __builtin_amdgcn_s_memrealtime();
    if (threadIdx.x == 0) {
      clock[0] = t0;
      clock[1] = t1;
      clock[2] = r0;
      clock[3] = r1;
    }
  }
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) sum += c[i][0];
  sink[static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x] = sum;
}

// Streaming read of `count` 16-byte words (non-temporal loads, 8 in flight
// per thread per step, grid-stride), one checksum word per thread written to
// sink (so the loads cannot be removed). One 256-thread block per compute
// unit keeps 8 MiB in flight on 256 CUs, which measured fastest: 4 loads in
// flight or more resident blocks per CU read 3-16% slower.
extern "C" __global__ __launch_bounds__(256) void xpu_peak_read(const xpu::u32x4 *__restrict__ input,
                                                                uint32_t *__restrict__ sink, uint64_t count) {
  const uint64_t tid = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  uint32_t acc = 0;
  uint64_t i = tid;
  for (; i + 7 * stride < count; i += 8 * stride) {
    xpu::u32x4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = xpu::load_nt16(input + i + u * stride);
#pragma unroll
    for (int u = 0; u < 8; ++u) acc ^= v[u].x ^ v[u].w;
  }
  for (; i < count; i += stride) {
    const xpu::u32x4 v = xpu::load_nt16(input + i);
    acc ^= v.x ^ v.w;
  }
  sink[tid] = acc;
}
