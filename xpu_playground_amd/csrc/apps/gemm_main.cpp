// Standalone gemm program (reference gemm.cpp:302-304).
#include "xpu_kernels.h"

int main(int argc, char **argv) { return run_gemm(argc, argv); }
