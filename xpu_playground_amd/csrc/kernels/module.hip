// Single gfx950 code object (xpu_kernels.hsaco) holding every kernel of the
// hot path, loaded at run time by the runtime with hipModuleLoadData.
#include "gemv.hip"
#include "synth.hip"
#include "qwen3_ops.hip"
#include "gemm.hip"
#include "peak.hip"
