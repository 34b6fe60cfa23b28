// Standalone Qwen3 decode program (reference qwen3/main.cpp:333-363).
#include "xpu_qwen3.h"

int main(int argc, char **argv) { return run_qwen3(argc, argv); }
