/*
 * xpu_runtime.hpp - header-only C++ wrapper over the C-ABI HIP runtime
 * (xpu_runtime.h) with the method set of the reference's
 * qwen3::LevelZeroRuntime (qwen3/level_zero_runtime.hpp:18-48), so that
 * host code written against that class compiles against this one with the
 * type name changed.
 *
 *   reference (level_zero_runtime.hpp)        this wrapper
 *   LevelZeroRuntime(module_path)        :21  HipRuntime(module_path)
 *   require_bmg_and_memory(bytes)        :26  require_device_and_memory(bytes)
 *                                             (require_bmg_and_memory kept as
 *                                              an alias of the same check)
 *   allocate_device(bytes, alignment)    :27  allocate_device(bytes, alignment)
 *   copy_to_device / copy_from_device  :28-29 same
 *   launch(fragment, work_items, args) :30-31 same (blocking, fragment match)
 *   device_name() / device_memory()    :32-33 same
 *   KernelArgument / kernel_argument() :13-16,50-52 same
 *
 * Errors: every failing C call is rethrown as std::runtime_error carrying the
 * call, file:line and xpu_last_error(), the way ZE_CHECK reports Level Zero
 * failures (level_zero_runtime.cpp:13-27). Non-copyable, single-threaded; the
 * runtime owns every allocation and frees them in the destructor
 * (level_zero_runtime.cpp:163-175).
 */
#ifndef XPU_RUNTIME_HPP
#define XPU_RUNTIME_HPP

#include "xpu_runtime.h"

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

namespace xpu {

struct KernelArgument {
  std::size_t size;
  const void *value;
};

template <typename T> KernelArgument kernel_argument(const T &value) {
  return KernelArgument{sizeof(T), &value};
}

inline void check_call(int status, const char *expr, const char *file, int line) {
  if (status == XPU_OK) return;
  throw std::runtime_error(std::string(expr) + " failed at " + file + ":" + std::to_string(line) +
                           " (status " + std::to_string(status) + "): " + xpu_last_error());
}

#define XPU_CHECK(expr) ::xpu::check_call((expr), #expr, __FILE__, __LINE__)

class HipRuntime {
public:
  explicit HipRuntime(const std::string &module_path, int device = -1) {
    XPU_CHECK(xpu_rt_create(module_path.empty() ? nullptr : module_path.c_str(), device, &rt_));
    char name[256];
    XPU_CHECK(xpu_rt_device_name(rt_, name, sizeof name));
    device_name_ = name;
    XPU_CHECK(xpu_rt_device_memory(rt_, &device_memory_));
  }
  ~HipRuntime() { xpu_rt_destroy(rt_); }
  HipRuntime(const HipRuntime &) = delete;
  HipRuntime &operator=(const HipRuntime &) = delete;

  // gfx950 and required_bytes + 512 MiB of free device memory.
  void require_device_and_memory(std::uint64_t required_bytes) const {
    XPU_CHECK(xpu_rt_require_device_and_memory(rt_, required_bytes));
  }
  void require_bmg_and_memory(std::uint64_t required_bytes) const {
    require_device_and_memory(required_bytes);
  }

  void *allocate_device(std::uint64_t bytes, std::uint64_t alignment = 4096) {
    void *p = nullptr;
    XPU_CHECK(xpu_rt_alloc(rt_, bytes, alignment, &p));
    return p;
  }
  void free_device(void *p) { XPU_CHECK(xpu_rt_free(rt_, p)); }
  void copy_to_device(void *destination, const void *source, std::size_t bytes) {
    XPU_CHECK(xpu_rt_copy_to_device(rt_, destination, source, bytes));
  }
  void copy_from_device(void *destination, const void *source, std::size_t bytes) {
    XPU_CHECK(xpu_rt_copy_from_device(rt_, destination, source, bytes));
  }
  void launch(const std::string &entry_fragment, std::uint32_t work_items,
              const std::vector<KernelArgument> &arguments) {
    std::vector<xpu_kernel_arg> args(arguments.size());
    for (std::size_t i = 0; i < arguments.size(); ++i) args[i] = {arguments[i].size, arguments[i].value};
    XPU_CHECK(xpu_rt_launch(rt_, entry_fragment.c_str(), work_items, args.data(),
                            static_cast<std::uint32_t>(args.size())));
  }
  void synchronize() { XPU_CHECK(xpu_rt_synchronize(rt_)); }

  const std::string &device_name() const { return device_name_; }
  std::uint64_t device_memory() const { return device_memory_; }
  xpu_runtime *handle() const { return rt_; }

private:
  xpu_runtime *rt_ = nullptr;
  std::string device_name_;
  std::uint64_t device_memory_ = 0;
};

}  // namespace xpu

#endif
