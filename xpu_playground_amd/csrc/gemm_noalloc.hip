// xpu_gemm_noalloc: the GEMM entry point for callers that cannot allocate
// device memory (code under HIP graph capture, tight serving loops). The
// FP32 split-K partials that xpu_gemm keeps in the runtime's grow-only
// workspace (outputs that leave most compute units idle, long reductions)
// go into `scratch`, a file-scope device array of fixed size that each GPU
// holds from the first runtime created on it until the process ends. Built
// by hipcc into the host library (host + gfx950 device code); the GEMM
// kernels themselves are those of the runtime's code object.
//
// `scratch` names a host-side stand-in in host code: its device address on
// each GPU comes from hipGetSymbolAddress, looked up once per device with
// that device current (xpu_rt_create), and only that address is passed to
// kernels. Every call on one GPU shares its array, which keeps the last
// call's contents; every partial a reduction reads is written by the same
// call first (each split's blocks store their whole tile range), so nothing
// needs clearing. Calls that overlap on one GPU (several runtimes or
// streams) race on the array.
#include "../../include/xpu_kernels.h"
#include "runtime_internal.hpp"

#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

namespace {

constexpr uint64_t kScratchBytes = XPU_GEMM_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mutex;
void *g_scratch_ptr[kMaxDevices] = {};

}  // namespace

namespace xpu {

int noalloc_scratch_setup(int device) {
  if (device < 0 || device >= kMaxDevices)
    return set_error(XPU_ERR_DEVICE, "xpu_gemm_noalloc supports device ids below " + std::to_string(kMaxDevices));
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[device]) return XPU_OK;
  void *ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !ptr)
    return set_error(XPU_ERR_HIP, hip_message(e, "hipGetSymbolAddress(scratch)", __FILE__, __LINE__));
  g_scratch_ptr[device] = ptr;
  return XPU_OK;
}

}  // namespace xpu

extern "C" int xpu_gemm_noalloc(xpu_runtime *rt, int dtype, const void *A, const void *B, void *C, uint32_t M,
                                uint32_t N, uint32_t K) {
  if (!rt) return xpu::set_error(XPU_ERR_INVALID, "xpu_gemm_noalloc: null runtime");
  if (rt->device < 0 || rt->device >= kMaxDevices || !g_scratch_ptr[rt->device])
    return xpu::set_error(XPU_ERR_DEVICE, "xpu_gemm_noalloc: no scratch address for this device");
  return xpu::gemm_run(rt, dtype, A, B, C, M, N, K, g_scratch_ptr[rt->device], kScratchBytes);
}
