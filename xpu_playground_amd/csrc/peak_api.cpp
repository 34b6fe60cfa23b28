// Peak-rate microbenchmarks (reference peak_compute_dpas.cpp and
// peak_mem_2d.cpp): the measured MFMA and HBM ceilings of the device the
// GEMM and GEMV rooflines are quoted against, plus the shader clock the
// MFMA loop actually ran at.
#include "../../include/xpu_kernels.h"
#include "host_common.hpp"
#include "runtime_internal.hpp"

#include <algorithm>
#include <cmath>
#include <iomanip>
#include <iostream>

using xpu::set_error;

namespace {

constexpr double kPeakMfmaBf16Tflops = 2500.0;  // MI355X dense bf16
constexpr double kPeakHbmGbs = 8000.0;          // MI355X HBM3E
constexpr uint32_t kMfmaFlops = 2 * 32 * 32 * 16;
constexpr uint32_t kChains = 8;

}  // namespace

extern "C" int xpu_peak_mfma(xpu_runtime *rt, const void *operand, void *sink, void *clock, uint32_t blocks,
                             uint32_t rounds) {
  if (!rt || !operand || !sink || !clock) return set_error(XPU_ERR_INVALID, "xpu_peak_mfma: null argument");
  if (blocks == 0 || rounds == 0) return set_error(XPU_ERR_INVALID, "xpu_peak_mfma: blocks and rounds must be positive");
  const xpu::KernelInfo *k = rt->find_exact("xpu_peak_mfma_bf16");
  if (!k) return set_error(XPU_ERR_NOT_FOUND, "kernel is absent from module: xpu_peak_mfma_bf16");
  const xpu_kernel_arg args[] = {{8, &operand}, {8, &sink}, {8, &clock}, {4, &rounds}};
  return rt->launch(*k, blocks, 1, 256, 0, args, 4);
}

extern "C" int xpu_peak_read(xpu_runtime *rt, const void *input, uint64_t bytes, void *sink, uint32_t blocks) {
  if (!rt || !input || !sink) return set_error(XPU_ERR_INVALID, "xpu_peak_read: null argument");
  if (bytes == 0 || bytes % 16 != 0 || reinterpret_cast<uintptr_t>(input) % 16 != 0 || blocks == 0)
    return set_error(XPU_ERR_INVALID, "xpu_peak_read: needs a 16-byte aligned, nonempty multiple of 16 bytes");
  const xpu::KernelInfo *k = rt->find_exact("xpu_peak_read");
  if (!k) return set_error(XPU_ERR_NOT_FOUND, "kernel is absent from module: xpu_peak_read");
  const uint64_t count = bytes / 16;
  const xpu_kernel_arg args[] = {{8, &input}, {8, &sink}, {8, &count}};
  return rt->launch(*k, blocks, 1, 256, 0, args, 3);
}

namespace {

void check(int rc) {
  if (rc) throw std::runtime_error(xpu_last_error());
}

struct RuntimeGuard {
  xpu_runtime *rt = nullptr;
  ~RuntimeGuard() { xpu_rt_destroy(rt); }
};

struct ComputeOptions {
  uint32_t waves_per_simd = 2;  // resident wavefronts per SIMD
  uint32_t rounds = 8192;       // peak_compute_dpas.cpp:24
  unsigned iterations = 100;
};

[[noreturn]] void compute_usage(const char *program, int status) {
  std::ostream &out = status ? std::cerr : std::cout;
  out << "Usage: " << program << " [--waves-per-simd N] [--rounds N] [--iterations N]\n"
      << "  --waves-per-simd N  wavefronts per SIMD (default: 2)\n"
      << "  --rounds N          eight-MFMA batches per wavefront (default: 8192)\n"
      << "  --iterations N      timed kernel launches (default: 100)\n";
  std::exit(status);
}

struct MemOptions {
  uint64_t size_mib = 4096;  // well above the 256 MiB last-level cache
  unsigned iterations = 100;  // peak_mem_2d.cpp:33
};

[[noreturn]] void mem_usage(const char *program, int status) {
  std::ostream &out = status ? std::cerr : std::cout;
  out << "Usage: " << program << " [--size-mib N] [--iterations N]\n"
      << "  --size-mib N    HBM read surface size (default: 4096)\n"
      << "  --iterations N  timed kernel launches (default: 100)\n";
  std::exit(status);
}

}  // namespace

extern "C" int run_peak_compute(int argc, char **argv) {
  try {
    ComputeOptions o;
    for (int i = 1; i < argc; ++i) {
      const std::string_view arg(argv[i]);
      if (arg == "-h" || arg == "--help") compute_usage(argv[0], 0);
      if (++i == argc) throw std::invalid_argument(std::string(arg) + " requires a value");
      const std::string_view value(argv[i]);
      if (arg == "--waves-per-simd") o.waves_per_simd = xpu::parse_positive<uint32_t>(value, arg);
      else if (arg == "--rounds") o.rounds = xpu::parse_positive<uint32_t>(value, arg);
      else if (arg == "--iterations") o.iterations = xpu::parse_positive<unsigned>(value, arg);
      else throw std::invalid_argument("unknown option: " + std::string(arg));
    }
    if (o.waves_per_simd > 2) throw std::invalid_argument("--waves-per-simd must be 1 or 2");
    RuntimeGuard guard;
    check(xpu_rt_create(nullptr, -1, &guard.rt));
    xpu_runtime *rt = guard.rt;
    std::cout << "Device: " << rt->name << " (" << rt->arch << ", " << rt->compute_units << " CUs)\n";
    int wall_khz = 0;
    if (hipDeviceGetAttribute(&wall_khz, hipDeviceAttributeWallClockRate, rt->device) != hipSuccess || wall_khz <= 0)
      throw std::runtime_error("cannot query the constant-rate clock frequency");
    // 256-thread blocks (4 wavefronts, one per SIMD), waves_per_simd per CU
    const uint32_t blocks = rt->compute_units * o.waves_per_simd;
    const uint64_t threads = static_cast<uint64_t>(blocks) * 256;
    void *operand = nullptr, *sink = nullptr, *clock = nullptr;
    check(xpu_rt_alloc(rt, 16, 256, &operand));
    check(xpu_rt_alloc(rt, threads * 4, 256, &sink));
    check(xpu_rt_alloc(rt, 32, 256, &clock));
    const uint16_t half[8] = {0x3f00, 0x3f00, 0x3f00, 0x3f00, 0x3f00, 0x3f00, 0x3f00, 0x3f00};  // bf16 0.5
    check(xpu_rt_copy_to_device(rt, operand, half, sizeof half));
    const double flops = static_cast<double>(threads / 64) * o.rounds * kChains * kMfmaFlops;
    std::cout << "MFMA shape: 32x32x16 BF16, " << kMfmaFlops << " FLOP/instruction\n"
              << "Launch: " << blocks << " blocks x 4 wavefronts x " << o.rounds << " rounds x " << kChains
              << " MFMA = " << std::fixed << std::setprecision(3) << flops / 1e12 << " TFLOP/launch\n";
    for (int i = 0; i < 3; ++i) check(xpu_peak_mfma(rt, operand, sink, clock, blocks, o.rounds));
    check(xpu_rt_synchronize(rt));
    void *start = nullptr, *stop = nullptr;
    check(xpu_rt_event_create(rt, &start));
    check(xpu_rt_event_create(rt, &stop));
    std::vector<double> tflops, mhz;
    for (unsigned i = 0; i < o.iterations; ++i) {
      check(xpu_rt_event_record(rt, start));
      check(xpu_peak_mfma(rt, operand, sink, clock, blocks, o.rounds));
      check(xpu_rt_event_record(rt, stop));
      float ms = 0;
      check(xpu_rt_event_elapsed_ms(start, stop, &ms));
      tflops.push_back(flops / (ms * 1e-3) / 1e12);
      uint64_t t[4];
      check(xpu_rt_copy_from_device(rt, t, clock, sizeof t));
      const double seconds = static_cast<double>(t[3] - t[2]) / (wall_khz * 1e3);
      if (seconds > 0) mhz.push_back(static_cast<double>(t[1] - t[0]) / seconds / 1e6);
    }
    xpu_rt_event_destroy(start);
    xpu_rt_event_destroy(stop);
    // checksum (peak_compute_dpas.cpp:196-206): every MFMA adds 16 * 0.25
    std::vector<float> s(threads);
    check(xpu_rt_copy_from_device(rt, s.data(), sink, threads * 4));
    const float expected = 28.0f + static_cast<float>(kChains) * o.rounds * 4.0f;
    const float tolerance = std::max(1.0f, expected * 1.0e-5f);
    for (float v : s)
      if (std::fabs(v - expected) > tolerance) throw std::runtime_error("MFMA checksum verification failed");
    const double med = xpu::median_of(tflops), best = xpu::max_of(tflops);
    const double clk = mhz.empty() ? 0.0 : xpu::median_of(mhz);
    std::cout << std::fixed << std::setprecision(2) << "Median BF16 compute: " << med << " TFLOP/s ("
              << 100.0 * med / kPeakMfmaBf16Tflops << "% of " << kPeakMfmaBf16Tflops << " TFLOP/s)\n"
              << "Best BF16 compute:   " << best << " TFLOP/s (" << 100.0 * best / kPeakMfmaBf16Tflops << "% of "
              << kPeakMfmaBf16Tflops << " TFLOP/s)\n"
              << "Shader clock during the loop: " << std::setprecision(0) << clk << " MHz (s_memtime over "
              << "s_memrealtime at " << wall_khz / 1000 << " MHz)\n"
              << "Checksum: PASS\n";
    return 0;
  } catch (const std::exception &error) {
    std::cerr << "Error: " << error.what() << '\n';
    return 1;
  }
}

extern "C" int run_peak_mem(int argc, char **argv) {
  try {
    MemOptions o;
    for (int i = 1; i < argc; ++i) {
      const std::string_view arg(argv[i]);
      if (arg == "-h" || arg == "--help") mem_usage(argv[0], 0);
      if (++i == argc) throw std::invalid_argument(std::string(arg) + " requires a value");
      const std::string_view value(argv[i]);
      if (arg == "--size-mib") o.size_mib = xpu::parse_positive<uint64_t>(value, arg);
      else if (arg == "--iterations") o.iterations = xpu::parse_positive<unsigned>(value, arg);
      else throw std::invalid_argument("unknown option: " + std::string(arg));
    }
    if (o.size_mib > (1ull << 20)) throw std::invalid_argument("--size-mib is too large");
    RuntimeGuard guard;
    check(xpu_rt_create(nullptr, -1, &guard.rt));
    xpu_runtime *rt = guard.rt;
    std::cout << "Device: " << rt->name << " (" << rt->arch << ", " << rt->compute_units << " CUs)\n";
    const uint64_t bytes = o.size_mib << 20;
    const uint32_t blocks = rt->compute_units;  // one block per CU (kernels/peak.hip)
    check(xpu_rt_require_device_and_memory(rt, bytes + blocks * 1024ull));
    void *input = nullptr, *sink = nullptr;
    check(xpu_rt_alloc(rt, bytes, 4096, &input));
    check(xpu_rt_alloc(rt, blocks * 1024ull, 256, &sink));
    check(xpu_fill_uniform(rt, XPU_DTYPE_BF16, input, bytes / 2, 7));
    check(xpu_rt_synchronize(rt));
    std::cout << "Surface: " << o.size_mib << " MiB, " << blocks << " blocks x 256 threads, 16-byte loads\n";
    for (int i = 0; i < 3; ++i) check(xpu_peak_read(rt, input, bytes, sink, blocks));
    check(xpu_rt_synchronize(rt));
    void *start = nullptr, *stop = nullptr;
    check(xpu_rt_event_create(rt, &start));
    check(xpu_rt_event_create(rt, &stop));
    std::vector<double> gbs;
    for (unsigned i = 0; i < o.iterations; ++i) {
      check(xpu_rt_event_record(rt, start));
      check(xpu_peak_read(rt, input, bytes, sink, blocks));
      check(xpu_rt_event_record(rt, stop));
      float ms = 0;
      check(xpu_rt_event_elapsed_ms(start, stop, &ms));
      gbs.push_back(static_cast<double>(bytes) / (ms * 1e-3) / 1e9);
    }
    xpu_rt_event_destroy(start);
    xpu_rt_event_destroy(stop);
    const double med = xpu::median_of(gbs), best = xpu::max_of(gbs);
    std::cout << std::fixed << std::setprecision(2) << "Median read bandwidth: " << med << " GB/s ("
              << 100.0 * med / kPeakHbmGbs << "% of " << kPeakHbmGbs << " GB/s)\n"
              << "Best read bandwidth:   " << best << " GB/s (" << 100.0 * best / kPeakHbmGbs << "% of "
              << kPeakHbmGbs << " GB/s)\n";
    return 0;
  } catch (const std::exception &error) {
    std::cerr << "Error: " << error.what() << '\n';
    return 1;
  }
}
