// Standalone gemm program (reference gemm.cpp:157-159).
#include "xpu_kernels.h"

int main(int argc, char **argv) { return run_gemm(argc, argv); }
