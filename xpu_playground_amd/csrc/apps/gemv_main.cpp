// Standalone gemv program (reference gemv.cpp:172-174).
#include "xpu_kernels.h"

int main(int argc, char **argv) { return run_gemv(argc, argv); }
