// Single gfx950 code object (xpu_kernels.hsaco) holding every kernel of the
// hot path, loaded at run time by the runtime with hipModuleLoadData.
#include "device_common.hpp"
#ifdef XPU_STAMPS
extern "C" __device__ uint32_t xpu_stamp_seq[xpu::kStampSlots];
extern "C" __device__ xpu::StampRecord xpu_stamp_ring[xpu::kStampSlots * xpu::kStampRing];
__device__ uint32_t xpu_stamp_seq[xpu::kStampSlots];
__device__ xpu::StampRecord xpu_stamp_ring[xpu::kStampSlots * xpu::kStampRing];
__device__ uint32_t xpu_stamp_phase[xpu::kPhaseSlots * xpu::kStampRing * xpu::kPhases];
#endif
#include "gemv.hip"
#include "synth.hip"
#include "qwen3_ops.hip"
#include "gemm.hip"
#include "prefill_attention.hip"
#include "peak.hip"
