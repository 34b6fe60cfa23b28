// Benchmark launcher with the modes of the reference's peak_sycl
// (peak_sycl.cpp:8-20,47-50): mem, compute, gemv, gemm. The reference
// execv()s a sibling program per mode; here each mode is an entry point of
// the same library, called in-process with the mode removed from argv.
#include "xpu_kernels.h"

#include <iostream>
#include <string>

namespace {

void usage(const char *program) {
  std::cout << "Usage:\n"
            << "  " << program << " mem [--size-mib N] [--iterations N]\n"
            << "  " << program << " compute [--waves-per-simd N] [--rounds N] [--iterations N]\n"
            << "  " << program << " gemv [--size N | --m M --k K] [--type bf16|fp16]\n"
            << "  " << program << " gemm [--size N | --m M --n N --k K] [--type bf16|fp16]\n";
}

}  // namespace

int main(int argc, char **argv) {
  if (argc < 2) {
    usage(argv[0]);
    std::cerr << "Error: missing benchmark mode\n";
    return 1;
  }
  const std::string mode = argv[1];
  if (mode == "-h" || mode == "--help") {
    usage(argv[0]);
    return 0;
  }
  argv[1] = argv[0];
  if (mode == "mem") return run_peak_mem(argc - 1, argv + 1);
  if (mode == "compute") return run_peak_compute(argc - 1, argv + 1);
  if (mode == "gemv") return run_gemv(argc - 1, argv + 1);
  if (mode == "gemm") return run_gemm(argc - 1, argv + 1);
  std::cerr << "Error: unknown benchmark mode: " << mode << '\n';
  return 1;
}
