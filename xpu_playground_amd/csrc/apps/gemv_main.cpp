// Standalone gemv program (reference gemv.cpp:237-239).
#include "xpu_kernels.h"

int main(int argc, char **argv) { return run_gemv(argc, argv); }
