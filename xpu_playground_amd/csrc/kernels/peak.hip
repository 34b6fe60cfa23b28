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

// ---- Synchronisation costs: what a dependent step between two groups of
// compute units costs on this device, in two forms.
//
// xpu_peak_empty: an empty kernel; a chain of dependent launches of it (one
// block per compute unit, on one stream or in a captured graph) measures the
// gap between the end of one kernel and the start of the next.
extern "C" __global__ __launch_bounds__(256) void xpu_peak_empty() {}

// xpu_peak_handoff_v<V>: `stages` all-to-all handoffs inside one cooperative
// launch of one block per compute unit. Each stage every block writes 64
// words of its own (stage-parity double buffered), publishes them, waits
// until every block has published, and checks 16 words of another block's
// output (mismatches set bit 2 of err[1]). V selects the publication:
//   0: every wave runs an agent-scope release fence, then the block barrier,
//      thread 0 stores its flag; wave 0 polls every flag, every wave runs an
//      agent-scope acquire fence (the C++-memory-model form)
//   1: every wave waits for its stores, the block barrier, then wave 0 alone
//      runs the release fence and stores the flag; wave 0 polls, runs the
//      acquire fence, block barrier
//   3: data written and read with agent-scope relaxed atomics (coherent at
//      the device, no cache maintenance), every wave waits for its stores,
//      barrier, thread 0 stores its flag; wave 0 polls
//   4: as 3, but each block adds 1 to the counter of its group of 32
//      blocks and wave 0 polls the group counters
// Every wait gives up after 1 << 20 polls and stops the grid (err[0]).
// times[b]: constant-clock ticks (100 MHz) block b spent in the stages.
namespace xpu {
XPU_DEVICE uint32_t peak_wave_min(uint32_t v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = min(v, static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), m)));
  return v;
}

template <int V>
XPU_DEVICE void peak_handoff(uint32_t *flags, uint32_t *counters, uint32_t *out, uint32_t *err, uint32_t stages,
                             uint64_t *times) {
  constexpr uint32_t kSpin = 1u << 20;
  constexpr bool kCoherent = V == 3 || V == 4, kCounters = V == 4;
  const uint32_t G = gridDim.x, b = blockIdx.x, tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t groups = (G + 31) / 32;
  __shared__ uint32_t status;
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  for (uint32_t s = 1; s <= stages; ++s) {
    uint32_t *mine = out + (s & 1u) * G * 64 + b * 64;
    const uint32_t value = s * 1000u + b;
    if (lane < 16) {
      if constexpr (kCoherent) __hip_atomic_store(mine + wave * 16 + lane, value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      else mine[wave * 16 + lane] = value;
    }
    if constexpr (V == 0) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
      __syncthreads();
      if (tid == 0) __hip_atomic_store(flags + b, s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      if (tid == 0) {
        if constexpr (V == 1) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        if constexpr (kCounters) __hip_atomic_fetch_add(counters + (b / 32) * 32, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else __hip_atomic_store(flags + b, s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    if (wave == 0) {
      uint32_t st = 0;
      for (uint32_t spin = 0;; ++spin) {
        bool ready;
        if constexpr (kCounters) {
          uint32_t ok = 1;
          if (lane < groups) {
            const uint32_t members = min(32u, G - lane * 32);
            ok = __hip_atomic_load(counters + lane * 32, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= members * s;
          }
          ready = peak_wave_min(ok) == 1;
        } else {
          uint32_t low = 0xffffffffu;
          for (uint32_t i = lane; i < G; i += 64)
            low = min(low, __hip_atomic_load(flags + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
          ready = peak_wave_min(low) >= s;
        }
        const uint32_t e = __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (ready) {
          st = 1;
          break;
        }
        if (e) {
          st = 2;
          break;
        }
        if (spin >= kSpin) {
          if (lane == 0) __hip_atomic_fetch_or(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          st = 2;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      if constexpr (V == 1) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      if (lane == 0) status = st;
    }
    __syncthreads();
    if (status != 1) return;
    if constexpr (V == 0) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    const uint32_t other = (b + 1 + wave) % G;
    const uint32_t *src = out + (s & 1u) * G * 64 + other * 64 + lane % 16;
    uint32_t v;
    if constexpr (kCoherent) v = __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else v = *src;
    if (lane < 16 && v != s * 1000u + other) __hip_atomic_fetch_or(err + 1, 4u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (tid == 0) times[b] = __builtin_amdgcn_s_memrealtime() - t0;
}
}  // namespace xpu

#define XPU_PEAK_HANDOFF(V)                                                                                  \
  extern "C" __global__ __launch_bounds__(256) void xpu_peak_handoff_v##V(                                  \
      uint32_t *flags, uint32_t *counters, uint32_t *out, uint32_t *err, uint32_t stages, uint64_t *times) { \
    xpu::peak_handoff<V>(flags, counters, out, err, stages, times);                                          \
  }
XPU_PEAK_HANDOFF(0)
XPU_PEAK_HANDOFF(1)
XPU_PEAK_HANDOFF(3)
XPU_PEAK_HANDOFF(4)
