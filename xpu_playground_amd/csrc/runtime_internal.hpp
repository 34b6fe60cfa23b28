// Internal definitions shared by the runtime and the entry-point libraries.
#pragma once

#include "../../include/xpu_runtime.h"

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace xpu {

int set_error(int code, const std::string &message);
void clear_error();
std::string hip_message(hipError_t e, const char *expr, const char *file, int line);

struct Geometry {
  uint32_t grid = 0, block = 0, shared = 0;
};

// Reference work-item convention (qwen3/level_zero_runtime.cpp:148-155,248):
// each launchable-by-fragment kernel derives its grid from the work-item
// count and, where needed, from its arguments. signature: one character per
// argument, p = pointer, q = 64-bit integer, u = 32-bit integer, f = float.
struct LaunchRule {
  const char *name;
  const char *signature;
  int (*geometry)(uint32_t work_items, const xpu_kernel_arg *args, const struct ::xpu_runtime &rt,
                  Geometry &g);
};

const LaunchRule *find_rule(const std::string &kernel_name);

struct KernelInfo {
  std::string name;
  hipFunction_t function = nullptr;
  const LaunchRule *rule = nullptr;
};

template <typename T> T arg_value(const xpu_kernel_arg *args, uint32_t index) {
  return *static_cast<const T *>(args[index].value);
}

// The GEMM launch behind xpu_gemm and xpu_gemm_noalloc: A and B are read in
// place; where K is split, the FP32 partials go to a workspace: the
// runtime's grow-only one when fixed_workspace is null, else
// fixed_workspace (fixed_capacity bytes; a larger need fails with
// XPU_ERR_INVALID before any launch).
int gemm_run(xpu_runtime *rt, int dtype, const void *A, const void *B, void *C, uint32_t M, uint32_t N, uint32_t K,
             void *fixed_workspace, uint64_t fixed_capacity);

// C = A W^T for W given [N][K], bf16, aligned operands (gemm_api.cpp);
// residual adds into C
// norm_w / Xn (optional): where the product goes through the split-K
// reduction, that kernel also writes Xn = RMSNorm(C) with gains norm_w and
// eps and sets *normed (N = 512 or 1024); otherwise
// *normed is false and the caller normalises.
int gemm_nt(xpu_runtime *rt, const void *A, const void *W, void *C, uint32_t M, uint32_t N, uint32_t K,
            bool residual, const void *norm_w = nullptr, void *Xn = nullptr, float eps = 0.0f,
            bool *normed = nullptr);
// The most workspace gemm_nt requests (its split-K partials), so a caller
// can reserve it once (xpu_runtime::scratch grows by synchronizing).
uint64_t gemm_nt_workspace_bound(const xpu_runtime *rt);

// Device address of the no-allocation scratch array on `device` (the
// current device), looked up once per device; called by xpu_rt_create.
int noalloc_scratch_setup(int device);

}  // namespace xpu

struct xpu_runtime {
  int device = -1;
  std::string name, arch, module_path;
  uint64_t total_memory = 0;
  uint32_t compute_units = 0, max_shared = 0;
  hipStream_t stream = nullptr;
  hipModule_t module = nullptr;
  std::vector<xpu::KernelInfo> kernels;
  std::map<void *, void *> allocations;
  // grow-only scratch for entry points that stage data (GEMM padding)
  void *workspace = nullptr;
  uint64_t workspace_bytes = 0;

  xpu_runtime() = default;
  xpu_runtime(const xpu_runtime &) = delete;
  xpu_runtime &operator=(const xpu_runtime &) = delete;
  ~xpu_runtime();
  const xpu::KernelInfo *find_exact(const std::string &name) const;
  // cooperative: every block resident at once (hipModuleLaunchCooperativeKernel
  // fails the launch otherwise), for kernels whose blocks wait on each other
  int launch(const xpu::KernelInfo &k, uint32_t gx, uint32_t gy, uint32_t bx, uint32_t shared,
             const xpu_kernel_arg *args, uint32_t nargs, bool cooperative = false);
  // at least `bytes` of device scratch, 256-byte aligned; contents undefined
  int scratch(uint64_t bytes, void **out);
};

#define XPU_HIP_RETURN(expr)                                                                 \
  do {                                                                                       \
    const hipError_t xpu_e_ = (expr);                                                        \
    if (xpu_e_ != hipSuccess)                                                                \
      return ::xpu::set_error(XPU_ERR_HIP, ::xpu::hip_message(xpu_e_, #expr, __FILE__, __LINE__)); \
  } while (0)
