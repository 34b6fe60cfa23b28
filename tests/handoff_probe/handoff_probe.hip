// Test-only probe (not part of the library or its programs): what one
// dependent step between kernels of one block per compute unit costs on
// this GPU, in two forms.
//
// 1. A kernel boundary: a chain of dependent launches of an empty kernel on
//    one stream and inside a captured graph; the time per launch is the gap
//    between the end of one kernel and the start of the next.
// 2. An all-to-all handoff inside one persistent (cooperative) launch, in
//    four publication forms (below).
//
// The Qwen3 decode step is a chain of such all-to-all steps (each GEMV
// needs the whole previous vector), so these figures decide between kernel
// boundaries and a persistent kernel. Built by __graft_entry__.build() into
// tests/handoff_probe/build/handoff_probe; run by tests/test_gpu_peak.py.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#define CHECK(expr)                                                                               \
  do {                                                                                            \
    const hipError_t e_ = (expr);                                                                 \
    if (e_ != hipSuccess) {                                                                       \
      std::fprintf(stderr, "Error: %s failed: %s (%s:%d)\n", #expr, hipGetErrorString(e_), __FILE__, \
                   __LINE__);                                                                     \
      std::exit(1);                                                                               \
    }                                                                                             \
  } while (0)

__global__ __launch_bounds__(256) void probe_empty() {}

// `stages` all-to-all handoffs inside one cooperative launch of one block
// per compute unit. Each stage every block writes 64 words of its own
// (stage-parity double buffered), publishes them, waits until every block
// has published, and checks 16 words of another block's output (mismatches
// set bit 2 of err[1]). V selects the publication:
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
// Every wait gives up after 1 << 20 polls and stops the grid (err[0]), so
// every wave exits. times[b]: constant-clock ticks block b spent in the
// stages.
__device__ uint32_t wave_min(uint32_t v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = min(v, static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), m)));
  return v;
}

template <int V>
__global__ __launch_bounds__(256) void probe_handoff(uint32_t *flags, uint32_t *counters, uint32_t *out,
                                                     uint32_t *err, uint32_t stages, uint64_t *times) {
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
      if constexpr (kCoherent)
        __hip_atomic_store(mine + wave * 16 + lane, value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      else
        mine[wave * 16 + lane] = value;
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
        if constexpr (kCounters)
          __hip_atomic_fetch_add(counters + (b / 32) * 32, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else
          __hip_atomic_store(flags + b, s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
          ready = wave_min(ok) == 1;
        } else {
          uint32_t low = 0xffffffffu;
          for (uint32_t i = lane; i < G; i += 64)
            low = min(low, __hip_atomic_load(flags + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
          ready = wave_min(low) >= s;
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
    if constexpr (kCoherent)
      v = __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
      v = *src;
    if (lane < 16 && v != s * 1000u + other)
      __hip_atomic_fetch_or(err + 1, 4u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (tid == 0) times[b] = __builtin_amdgcn_s_memrealtime() - t0;
}

static unsigned positive(const char *text, const char *opt) {
  char *end = nullptr;
  const unsigned long v = std::strtoul(text, &end, 10);
  if (!*text || *end || v == 0 || v > 1000000) {
    std::fprintf(stderr, "Error: %s requires a positive integer up to 1000000\n", opt);
    std::exit(1);
  }
  return static_cast<unsigned>(v);
}

int main(int argc, char **argv) {
  unsigned launches = 2000, stages = 500;
  for (int i = 1; i < argc; i += 2) {
    if (i + 1 >= argc) {
      std::fprintf(stderr, "Error: %s requires a value\n", argv[i]);
      return 1;
    }
    if (!std::strcmp(argv[i], "--launches")) launches = positive(argv[i + 1], argv[i]);
    else if (!std::strcmp(argv[i], "--stages")) stages = positive(argv[i + 1], argv[i]);
    else {
      std::fprintf(stderr, "Error: unknown option: %s\n", argv[i]);
      return 1;
    }
  }
  int dev = 0;
  CHECK(hipSetDevice(dev));
  hipDeviceProp_t prop;
  CHECK(hipGetDeviceProperties(&prop, dev));
  int coop = 0, wall_khz = 0;
  CHECK(hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev));
  CHECK(hipDeviceGetAttribute(&wall_khz, hipDeviceAttributeWallClockRate, dev));
  if (!coop || wall_khz <= 0) {
    std::fprintf(stderr, "Error: the device lacks cooperative launch or a constant-rate clock\n");
    return 1;
  }
  const uint32_t G = static_cast<uint32_t>(prop.multiProcessorCount);
  std::printf("Device: %s (%s, %u CUs)\n", prop.name, prop.gcnArchName, G);

  hipStream_t stream;
  CHECK(hipStreamCreate(&stream));
  hipEvent_t start, stop;
  CHECK(hipEventCreate(&start));
  CHECK(hipEventCreate(&stop));
  auto chain = [&] {
    for (unsigned i = 0; i < launches; ++i) hipLaunchKernelGGL(probe_empty, dim3(G), dim3(256), 0, stream);
    CHECK(hipGetLastError());
  };
  chain();
  CHECK(hipStreamSynchronize(stream));
  CHECK(hipEventRecord(start, stream));
  chain();
  CHECK(hipEventRecord(stop, stream));
  CHECK(hipEventSynchronize(stop));
  float ms = 0;
  CHECK(hipEventElapsedTime(&ms, start, stop));
  const double stream_us = ms * 1e3 / launches;
  hipGraph_t graph;
  hipGraphExec_t exec;
  CHECK(hipStreamBeginCapture(stream, hipStreamCaptureModeGlobal));
  chain();
  CHECK(hipStreamEndCapture(stream, &graph));
  CHECK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
  CHECK(hipGraphLaunch(exec, stream));
  CHECK(hipStreamSynchronize(stream));
  CHECK(hipEventRecord(start, stream));
  CHECK(hipGraphLaunch(exec, stream));
  CHECK(hipEventRecord(stop, stream));
  CHECK(hipEventSynchronize(stop));
  CHECK(hipEventElapsedTime(&ms, start, stop));
  CHECK(hipGraphExecDestroy(exec));
  CHECK(hipGraphDestroy(graph));
  const double graph_us = ms * 1e3 / launches;
  std::printf("Kernel boundary, %u blocks per launch: %.3f us per dependent launch on a stream, %.3f us in a graph\n",
              G, stream_us, graph_us);

  const uint32_t groups = (G + 31) / 32;
  uint32_t *flags, *counters, *out, *err;
  uint64_t *times;
  CHECK(hipMalloc(&flags, G * 4ull));
  CHECK(hipMalloc(&counters, groups * 32 * 4ull));
  CHECK(hipMalloc(&out, 2ull * G * 64 * 4));
  CHECK(hipMalloc(&err, 8));
  CHECK(hipMalloc(&times, G * 8ull));
  typedef void (*Kernel)(uint32_t *, uint32_t *, uint32_t *, uint32_t *, uint32_t, uint64_t *);
  const Kernel kernels[] = {probe_handoff<0>, probe_handoff<1>, probe_handoff<3>, probe_handoff<4>};
  const char *labels[] = {"fences in every wave (C++ release/acquire)", "one fence pair per block",
                          "device-coherent data, flag per block", "device-coherent data, counter per 32 blocks"};
  bool data_ok = true;
  for (int i = 0; i < 4; ++i) {
    // one block per CU must be co-resident for the waits to complete
    int per_cu = 0;
    CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(kernels[i]), 256, 0));
    if (per_cu < 1) {
      std::fprintf(stderr, "Error: the handoff kernel cannot keep one block per CU resident\n");
      return 1;
    }
    CHECK(hipMemsetAsync(flags, 0, G * 4ull, stream));
    CHECK(hipMemsetAsync(counters, 0, groups * 32 * 4ull, stream));
    CHECK(hipMemsetAsync(out, 0, 2ull * G * 64 * 4, stream));
    CHECK(hipMemsetAsync(err, 0, 8, stream));
    void *args[] = {&flags, &counters, &out, &err, &stages, &times};
    CHECK(hipLaunchCooperativeKernel(reinterpret_cast<const void *>(kernels[i]), dim3(G), dim3(256), args, 0, stream));
    CHECK(hipStreamSynchronize(stream));
    uint32_t e[2] = {0, 0};
    CHECK(hipMemcpy(e, err, 8, hipMemcpyDeviceToHost));
    if (e[0]) {
      std::fprintf(stderr, "Error: %s: a wait passed its bound\n", labels[i]);
      return 1;
    }
    if (e[1]) data_ok = false;
    std::vector<uint64_t> t(G);
    CHECK(hipMemcpy(t.data(), times, G * 8ull, hipMemcpyDeviceToHost));
    const uint64_t slowest = *std::max_element(t.begin(), t.end());
    std::printf("In-kernel all-to-all handoff, %s: %.3f us per stage\n", labels[i],
                slowest / (wall_khz * 1e-3) / stages);
  }
  CHECK(hipFree(flags));
  CHECK(hipFree(counters));
  CHECK(hipFree(out));
  CHECK(hipFree(err));
  CHECK(hipFree(times));
  CHECK(hipEventDestroy(start));
  CHECK(hipEventDestroy(stop));
  CHECK(hipStreamDestroy(stream));
  std::printf("Data check: %s\n", data_ok ? "PASS" : "FAIL");
  return data_ok ? 0 : 1;
}
