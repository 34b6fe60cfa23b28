// GEMV entry points: xpu_gemv (kernel launch), the device fills, and the
// run_gemv command-line program (reference gemv.cpp and the GEMV mode of
// level_zero/peak_l0.cpp:811-893).
#include "../../include/xpu_kernels.h"
#include "host_common.hpp"
#include "runtime_internal.hpp"

#include <cstdio>
#include <cstdlib>
#include <iomanip>
#include <iostream>
#include <sstream>

namespace xpu {

// Launch geometry of the GEMV kernels (kernels/gemv.hip): 256 threads, R rows
// per wavefront, a grid-stride loop over 4R-row tiles.
struct GemvPlan {
  std::string kernel;
  uint32_t grid = 0, shared = 0;
};

int plan_gemv(const xpu_runtime &rt, int dtype, const void *A, const void *x, uint32_t M,
              uint32_t K, uint64_t lda, GemvPlan &plan) {
  const bool vec = (reinterpret_cast<uintptr_t>(A) % 16 == 0) &&
                   (reinterpret_cast<uintptr_t>(x) % 16 == 0) && K % 8 == 0 && lda % 8 == 0;
  const uint64_t kpad = (static_cast<uint64_t>(K) + 511u) & ~uint64_t{511};
  const bool global_x = kpad * 2 > rt.max_shared;
  if (global_x && !vec)
    return set_error(XPU_ERR_INVALID, "GEMV K=" + std::to_string(K) +
                                          " exceeds the LDS and needs 16-byte aligned A, x and K, lda "
                                          "multiples of 8");
  // rows per wavefront and 512-column chunks per pipelined load batch. With
  // the vector in LDS: rows longer than 8192 columns one per wavefront, 4
  // chunks per batch (6.7 TB/s at 16384^2 fp16, against 5.8-6.2 for 2 rows);
  // shorter rows two per wavefront, 2 chunks per batch, so the bubble at each
  // row's end is shared by two rows (6.6 TB/s at 65536 x 4096 and
  // 32768 x 8192, against 5.2 and 6.3 for one row). 8 chunks when the vector
  // is read from global memory, 2 for the 16-bit-load path of unaligned
  // operands.
  const bool short_rows = vec && !global_x && K <= 8192;
  const uint32_t rows = short_rows ? 2 : 1, unroll = !vec ? 2 : global_x ? 8 : short_rows ? 2 : 4;
  plan.shared = global_x ? 0 : static_cast<uint32_t>(kpad * 2);
  // one block per compute unit, grid-stride over 4-row tiles: each block
  // stages the vector once
  const uint64_t tiles = (static_cast<uint64_t>(M) + 4 * rows - 1) / (4 * rows);
  plan.grid = static_cast<uint32_t>(std::min<uint64_t>(tiles, rt.compute_units));
  plan.kernel = std::string("xpu_gemv_") + (dtype ? "fp16" : "bf16") + "_r" + std::to_string(rows) + "u" +
                std::to_string(unroll) + (vec ? (global_x ? "_vecg" : "_vec") : "_any");
  return XPU_OK;
}

}  // namespace xpu

using xpu::set_error;

extern "C" int xpu_gemv(xpu_runtime *rt, int dtype, const void *A, const void *x, void *y,
                        uint32_t M, uint32_t K, uint64_t lda) {
  if (!rt || !A || !x || !y) return set_error(XPU_ERR_INVALID, "xpu_gemv: null argument");
  if (dtype != XPU_DTYPE_BF16 && dtype != XPU_DTYPE_FP16)
    return set_error(XPU_ERR_INVALID, "xpu_gemv: dtype must be bf16 (0) or fp16 (1)");
  if (M == 0 || K == 0) return set_error(XPU_ERR_INVALID, "xpu_gemv: M and K must be positive");
  if (lda < K) return set_error(XPU_ERR_INVALID, "xpu_gemv: lda must be >= K");
  xpu::GemvPlan plan;
  int rc = xpu::plan_gemv(*rt, dtype, A, x, M, K, lda, plan);
  if (rc) return rc;
  const xpu::KernelInfo *k = rt->find_exact(plan.kernel);
  if (!k) return set_error(XPU_ERR_NOT_FOUND, "kernel is absent from module: " + plan.kernel);
  const xpu_kernel_arg args[] = {{8, &A}, {8, &x}, {8, &y}, {4, &M}, {4, &K}, {8, &lda}};
  return rt->launch(*k, plan.grid, 1, 256, plan.shared, args, 6);
}

extern "C" int xpu_fill_uniform(xpu_runtime *rt, int dtype, void *dst, uint64_t count, uint64_t seed) {
  if (!rt || !dst) return set_error(XPU_ERR_INVALID, "xpu_fill_uniform: null argument");
  if (count == 0) return XPU_OK;
  const xpu::KernelInfo *k = rt->find_exact("xpu_fill_uniform_u16");
  if (!k) return set_error(XPU_ERR_NOT_FOUND, "kernel is absent from module: xpu_fill_uniform_u16");
  const uint64_t mixed = xpu::mix64(seed);
  const uint32_t dt = static_cast<uint32_t>(dtype);
  const uint32_t grid = static_cast<uint32_t>(std::min<uint64_t>((count + 255) / 256, 65536));
  const xpu_kernel_arg args[] = {{8, &dst}, {8, &count}, {8, &mixed}, {4, &dt}};
  return rt->launch(*k, grid, 1, 256, 0, args, 4);
}

extern "C" int xpu_fill_reference_gemv(xpu_runtime *rt, int dtype, void *matrix, void *vector,
                                       uint32_t m, uint32_t k, uint32_t ld) {
  if (!rt || !matrix || !vector) return set_error(XPU_ERR_INVALID, "null argument");
  if (ld < k || m == 0) return set_error(XPU_ERR_INVALID, "invalid reference fill shape");
  const xpu::KernelInfo *kern = rt->find_exact("xpu_fill_reference_gemv");
  if (!kern) return set_error(XPU_ERR_NOT_FOUND, "kernel is absent from module: xpu_fill_reference_gemv");
  const uint32_t dt = static_cast<uint32_t>(dtype);
  const uint64_t total = static_cast<uint64_t>(m) * ld;
  const uint32_t grid = static_cast<uint32_t>(std::min<uint64_t>((total + 255) / 256, 65536));
  const xpu_kernel_arg args[] = {{8, &matrix}, {8, &vector}, {4, &m}, {4, &k}, {4, &ld}, {4, &dt}};
  return rt->launch(*kern, grid, 1, 256, 0, args, 6);
}

// ---------------------------------------------------------------- run_gemv

namespace {

struct GemvOptions {
  uint32_t m = 16384, k = 16384;          // gemv.cpp:21
  unsigned iterations = 50, warmups = 5;  // gemv.cpp:22
  int dtype = XPU_DTYPE_BF16;
  // gemv.cpp:91-103: the reference's hash initialisation is its only input,
  // so it is the default here too; --init uniform selects the seeded
  // U[-1,1] data of the benchmark configurations
  bool reference_init = true;
  uint64_t seed = 1;
  uint32_t rotate = 1;                    // distinct copies of A cycled by the timed loop
  uint32_t check_rows = 64;               // gemv.cpp:119 checks min(M, 64) rows
};

[[noreturn]] void gemv_usage(const char *program, int status) {
  std::ostream &out = status ? std::cerr : std::cout;
  out << "Usage: " << program << " [--size N | --m M --k K] [--type bf16|fp16]\n"
      << "       [--iterations N] [--warmups N] [--init reference|uniform] [--seed N]\n"
      << "       [--rotate N] [--check-rows N]\n";
  std::exit(status);
}

// gemv.cpp:45-64
GemvOptions parse_gemv(int argc, char **argv) {
  GemvOptions o;
  for (int i = 1; i < argc; ++i) {
    const std::string_view arg(argv[i]);
    if (arg == "-h" || arg == "--help") gemv_usage(argv[0], 0);
    if (++i == argc) throw std::invalid_argument(std::string(arg) + " requires a value");
    const std::string_view value(argv[i]);
    if (arg == "--size") o.m = o.k = xpu::parse_positive<uint32_t>(value, arg);
    else if (arg == "--m") o.m = xpu::parse_positive<uint32_t>(value, arg);
    else if (arg == "--k") o.k = xpu::parse_positive<uint32_t>(value, arg);
    else if (arg == "--iterations") o.iterations = xpu::parse_positive<unsigned>(value, arg);
    else if (arg == "--warmups") o.warmups = xpu::parse_positive<unsigned>(value, arg);
    else if (arg == "--type" && value == "fp16") o.dtype = XPU_DTYPE_FP16;
    else if (arg == "--type" && value == "bf16") o.dtype = XPU_DTYPE_BF16;
    else if (arg == "--type") throw std::invalid_argument("--type must be bf16 or fp16");
    else if (arg == "--init" && value == "uniform") o.reference_init = false;
    else if (arg == "--init" && value == "reference") o.reference_init = true;
    else if (arg == "--init") throw std::invalid_argument("--init must be uniform or reference");
    else if (arg == "--seed") o.seed = xpu::parse_unsigned<uint64_t>(value, arg);
    else if (arg == "--rotate") o.rotate = xpu::parse_positive<uint32_t>(value, arg);
    else if (arg == "--check-rows") o.check_rows = xpu::parse_unsigned<uint32_t>(value, arg);
    else throw std::invalid_argument("unknown option: " + std::string(arg));
  }
  return o;
}

void check(int rc) {
  if (rc) throw std::runtime_error(xpu_last_error());
}

struct RuntimeGuard {
  xpu_runtime *rt = nullptr;
  ~RuntimeGuard() { xpu_rt_destroy(rt); }
};

}  // namespace

extern "C" int run_gemv(int argc, char **argv) {
  try {
    const GemvOptions o = parse_gemv(argc, argv);
    RuntimeGuard guard;
    check(xpu_rt_create(nullptr, -1, &guard.rt));
    xpu_runtime *rt = guard.rt;
    std::cout << "Device: " << rt->name << " (" << rt->arch << ", " << rt->compute_units
              << " CUs)\n";
    // The reference hashes the linear index of its matrix padded to 32
    // columns (gemv.cpp:79-80,91-98); with the same row stride here every
    // element gets the reference's value. The product still covers K columns
    // only: the reference's padding columns keep hash data and enter its sum
    // when K % 32 != 0, which is the reference's bug, not its contract.
    const uint64_t ld64 = o.reference_init ? (static_cast<uint64_t>(o.k) + 31u) / 32u * 32u : o.k;
    if (ld64 > UINT32_MAX) throw std::overflow_error("matrix dimension is too large");
    const uint32_t ld = static_cast<uint32_t>(ld64);
    const uint64_t matrix_bytes = static_cast<uint64_t>(o.m) * ld * 2;
    check(xpu_rt_require_device_and_memory(rt, matrix_bytes * o.rotate + (o.k + o.m) * 4ull));
    std::vector<void *> matrices(o.rotate);
    void *x = nullptr, *y = nullptr;
    for (auto &a : matrices) check(xpu_rt_alloc(rt, matrix_bytes, 256, &a));
    check(xpu_rt_alloc(rt, o.k * 2ull, 256, &x));
    check(xpu_rt_alloc(rt, o.m * 2ull, 256, &y));
    for (uint32_t c = 0; c < o.rotate; ++c) {
      if (o.reference_init) check(xpu_fill_reference_gemv(rt, o.dtype, matrices[c], x, o.m, o.k, ld));
      else check(xpu_fill_uniform(rt, o.dtype, matrices[c], static_cast<uint64_t>(o.m) * o.k, o.seed + c));
    }
    if (!o.reference_init)
      check(xpu_fill_uniform(rt, o.dtype, x, o.k, o.seed + 0x5bd1e995ull));
    check(xpu_rt_memset(rt, y, 0, o.m * 2ull));
    check(xpu_rt_synchronize(rt));

    void *start = nullptr, *stop = nullptr;
    check(xpu_rt_event_create(rt, &start));
    check(xpu_rt_event_create(rt, &stop));
    for (unsigned i = 0; i < o.warmups; ++i)
      check(xpu_gemv(rt, o.dtype, matrices[i % o.rotate], x, y, o.m, o.k, ld));
    check(xpu_rt_synchronize(rt));
    // gemv.cpp:109-118: one timed launch per iteration; the reference counts
    // 2*M*K FLOP and 2*M*K matrix bytes (:109-110)
    const double flops = 2.0 * o.m * o.k;
    const double ref_bytes = 2.0 * o.m * o.k;
    const double alg_bytes = ref_bytes + 2.0 * o.k + 2.0 * o.m;
    std::vector<double> rates, bandwidths, alg_bandwidths, times;
    for (unsigned i = 0; i < o.iterations; ++i) {
      check(xpu_rt_event_record(rt, start));
      check(xpu_gemv(rt, o.dtype, matrices[(o.warmups + i) % o.rotate], x, y, o.m, o.k, ld));
      check(xpu_rt_event_record(rt, stop));
      float ms = 0;
      check(xpu_rt_event_elapsed_ms(start, stop, &ms));
      const double s = ms * 1e-3;
      times.push_back(s);
      rates.push_back(flops / s / 1e9);
      bandwidths.push_back(ref_bytes / s / 1e9);
      alg_bandwidths.push_back(alg_bytes / s / 1e9);
    }
    xpu_rt_event_destroy(start);
    xpu_rt_event_destroy(stop);
    // the last timed launch used matrices[(warmups + iterations - 1) % rotate]
    const void *checked = matrices[(o.warmups + o.iterations - 1) % o.rotate];

    // Verification (gemv.cpp:119-134): the first min(M, check_rows) rows
    // against a sequential FP32 host sum (tolerance max(1, 1%)), plus FP64
    // error statistics in units of the output type's ulp.
    const uint32_t rows = std::min(o.m, o.check_rows);
    double err2 = 0, ref2 = 0, max_ulps = 0;
    if (rows) {
      std::vector<uint16_t> hy(rows), ha(static_cast<size_t>(rows) * ld), hx(o.k);
      check(xpu_rt_copy_from_device(rt, hy.data(), y, rows * 2ull));
      check(xpu_rt_copy_from_device(rt, ha.data(), checked, ha.size() * 2));
      check(xpu_rt_copy_from_device(rt, hx.data(), x, o.k * 2ull));
      std::vector<float> xf(o.k);
      for (uint32_t c = 0; c < o.k; ++c) xf[c] = xpu::decode16(hx[c], o.dtype);
      for (uint32_t r = 0; r < rows; ++r) {
        float expected = 0.0f;
        double exact = 0.0;
        for (uint32_t c = 0; c < o.k; ++c) {
          const float a = xpu::decode16(ha[static_cast<size_t>(r) * ld + c], o.dtype);
          expected += a * xf[c];
          exact += static_cast<double>(a) * xf[c];
        }
        const float actual = xpu::decode16(hy[r], o.dtype);
        if (std::fabs(actual - expected) > std::max(1.0f, std::fabs(expected) * 0.01f))
          throw std::runtime_error("GEMV verification failed");  // gemv.cpp:135-136
        // error against the accumulated value rounded to the output type
        const double ref = xpu::decode16(xpu::encode16(static_cast<float>(exact), o.dtype), o.dtype);
        err2 += (actual - ref) * (actual - ref);
        ref2 += ref * ref;
        const double ulp = o.dtype ? xpu::fp16_ulp(ref) : xpu::bf16_ulp(ref);
        max_ulps = std::max(max_ulps, std::fabs(actual - ref) / ulp);
      }
    }
    const double rel_l2 = ref2 > 0 ? std::sqrt(err2 / ref2) : std::sqrt(err2);
    const double med_alg = xpu::median_of(alg_bandwidths);
    std::cout << "Type: " << (o.dtype ? "FP16" : "BF16") << ", shape: " << o.m << 'x' << o.k
              << '\n';
    if (o.reference_init)
      std::cout << "Input: reference hash (gemv.cpp:91-103), row stride " << ld << '\n';
    else
      std::cout << "Input: uniform [-1,1), seed " << o.seed << '\n';
    std::cout << std::fixed << std::setprecision(2) << "Median: " << xpu::median_of(rates)
              << " GFLOP/s, " << xpu::median_of(bandwidths) << " GB/s\n"
              << "Best:   " << xpu::max_of(rates) << " GFLOP/s, " << xpu::max_of(bandwidths)
              << " GB/s\n"
              << "HBM roofline: " << med_alg << " GB/s of A+x+y traffic = " << (med_alg / 8000.0 * 100.0)
              << "% of 8000 GB/s (median " << xpu::median_of(times) * 1e6 << " us)\n"
              << std::scientific << std::setprecision(3) << "Accuracy: rel-L2 " << rel_l2
              << ", max " << std::fixed << std::setprecision(2) << max_ulps
              << " ulp vs the FP64 sum rounded to the output type, over "
              << rows << " rows\n"
              << "Verification: PASS\n";
    return 0;
  } catch (const std::exception &error) {
    std::cerr << "Error: " << error.what() << '\n';
    return 1;
  }
}
