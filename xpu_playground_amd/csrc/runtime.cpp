// C-ABI HIP runtime for gfx950 (include/xpu_runtime.h).
//
// Replaces the reference's Level Zero runtime (qwen3/level_zero_runtime.cpp):
// device selection (:52-84) becomes hipSetDevice + gcnArchName check,
// zeModuleCreate (:119-147) becomes hipModuleLoad of a gfx950 code object,
// zeModuleGetKernelNames (:148-160) becomes a walk of the code object's ELF
// symbol table, zeKernelSetArgumentValue + zeCommandListAppendLaunchKernel
// (:225-255) becomes hipModuleLaunchKernel on one default-priority stream,
// kernel timestamps become hipEvents.
#include "../../include/xpu_runtime.h"
#include "runtime_internal.hpp"

#include <dlfcn.h>
#include <elf.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <sstream>
#include <string>
#include <vector>

namespace {

thread_local std::string g_last_error;

}  // namespace

namespace xpu {

int set_error(int code, const std::string &message) {
  g_last_error = message;
  return code;
}

void clear_error() { g_last_error.clear(); }

std::string hip_message(hipError_t e, const char *expr, const char *file, int line) {
  std::ostringstream out;
  out << expr << " failed at " << file << ':' << line << " (HIP error " << static_cast<int>(e)
      << ": " << hipGetErrorName(e) << ')';
  return out.str();
}

namespace {

// Kernel names of a code object: symbols whose name ends in ".kd" are AMDGPU
// kernel descriptors, one per __global__ function.
std::vector<std::string> elf_kernel_names(const std::vector<char> &image) {
  std::vector<std::string> names;
  if (image.size() < sizeof(Elf64_Ehdr)) return names;
  const auto *eh = reinterpret_cast<const Elf64_Ehdr *>(image.data());
  if (std::memcmp(eh->e_ident, ELFMAG, SELFMAG) != 0 || eh->e_ident[EI_CLASS] != ELFCLASS64)
    return names;
  if (eh->e_shoff == 0 || eh->e_shoff + uint64_t(eh->e_shnum) * sizeof(Elf64_Shdr) > image.size())
    return names;
  const auto *sh = reinterpret_cast<const Elf64_Shdr *>(image.data() + eh->e_shoff);
  for (unsigned i = 0; i < eh->e_shnum; ++i) {
    if (sh[i].sh_type != SHT_SYMTAB && sh[i].sh_type != SHT_DYNSYM) continue;
    if (sh[i].sh_link >= eh->e_shnum) continue;
    const Elf64_Shdr &strtab = sh[sh[i].sh_link];
    if (sh[i].sh_offset + sh[i].sh_size > image.size() ||
        strtab.sh_offset + strtab.sh_size > image.size() || sh[i].sh_entsize != sizeof(Elf64_Sym))
      continue;
    const auto *sym = reinterpret_cast<const Elf64_Sym *>(image.data() + sh[i].sh_offset);
    const size_t count = sh[i].sh_size / sizeof(Elf64_Sym);
    for (size_t s = 0; s < count; ++s) {
      if (sym[s].st_name >= strtab.sh_size) continue;
      const char *name = image.data() + strtab.sh_offset + sym[s].st_name;
      const size_t len = strnlen(name, strtab.sh_size - sym[s].st_name);
      if (len > 3 && std::strncmp(name + len - 3, ".kd", 3) == 0) {
        std::string kernel(name, len - 3);
        if (std::find(names.begin(), names.end(), kernel) == names.end()) names.push_back(kernel);
      }
    }
  }
  return names;
}

}  // namespace

std::string library_directory() {
  Dl_info info{};
  if (dladdr(reinterpret_cast<void *>(&xpu_rt_create), &info) && info.dli_fname) {
    std::string path(info.dli_fname);
    const auto slash = path.find_last_of('/');
    return slash == std::string::npos ? "." : path.substr(0, slash);
  }
  return ".";
}

}  // namespace xpu

xpu_runtime::~xpu_runtime() {
  // teardown: errors cannot be reported from a destructor
  if (device >= 0) (void)hipSetDevice(device);
  if (stream) (void)hipStreamSynchronize(stream);
  for (auto &entry : allocations) (void)hipFree(entry.second);
  if (workspace) (void)hipFree(workspace);
  if (module) (void)hipModuleUnload(module);
  if (stream) (void)hipStreamDestroy(stream);
}

const xpu::KernelInfo *xpu_runtime::find_exact(const std::string &name) const {
  for (const auto &k : kernels)
    if (k.name == name) return &k;
  return nullptr;
}

int xpu_runtime::scratch(uint64_t bytes, void **out) {
  if (bytes > workspace_bytes) {
    XPU_HIP_RETURN(hipSetDevice(device));
    if (workspace) {
      // earlier launches on the stream may still read the old block
      XPU_HIP_RETURN(hipStreamSynchronize(stream));
      XPU_HIP_RETURN(hipFree(workspace));
      workspace = nullptr;
      workspace_bytes = 0;
    }
    XPU_HIP_RETURN(hipMalloc(&workspace, bytes));
    workspace_bytes = bytes;
  }
  *out = workspace;
  return XPU_OK;
}

int xpu_runtime::launch(const xpu::KernelInfo &k, uint32_t gx, uint32_t gy, uint32_t bx,
                        uint32_t shared, const xpu_kernel_arg *args, uint32_t nargs, bool cooperative) {
  using xpu::set_error;
  if (gx == 0 || gy == 0 || bx == 0 || bx > 1024)
    return set_error(XPU_ERR_INVALID, "invalid launch geometry for " + k.name);
  if (shared > max_shared)
    return set_error(XPU_ERR_INVALID, "kernel " + k.name + " needs " + std::to_string(shared) +
                                          " bytes of LDS, device allows " +
                                          std::to_string(max_shared));
  void *params[32];
  if (nargs > 32) return set_error(XPU_ERR_INVALID, "too many kernel arguments");
  for (uint32_t i = 0; i < nargs; ++i) {
    if (!args[i].value || args[i].size == 0)
      return set_error(XPU_ERR_INVALID, "null kernel argument " + std::to_string(i));
    params[i] = const_cast<void *>(args[i].value);
  }
  if (cooperative)
    XPU_HIP_RETURN(hipModuleLaunchCooperativeKernel(k.function, gx, gy, 1, bx, 1, 1, shared, stream, params));
  else
    XPU_HIP_RETURN(hipModuleLaunchKernel(k.function, gx, gy, 1, bx, 1, 1, shared, stream, params, nullptr));
  return XPU_OK;
}

using xpu::clear_error;
using xpu::set_error;

extern "C" {

const char *xpu_last_error(void) { return g_last_error.c_str(); }

int xpu_rt_create(const char *module_path, int device, xpu_runtime **out) {
  if (!out) return set_error(XPU_ERR_INVALID, "xpu_rt_create: null output");
  *out = nullptr;
  clear_error();
  int count = 0;
  XPU_HIP_RETURN(hipGetDeviceCount(&count));
  if (count <= 0) return set_error(XPU_ERR_DEVICE, "no HIP device is visible");
  if (device < 0) {
    const char *env = std::getenv("XPU_DEVICE");
    device = env ? std::atoi(env) : 0;
  }
  if (device >= count)
    return set_error(XPU_ERR_DEVICE, "HIP device " + std::to_string(device) + " does not exist");
  auto rt = std::make_unique<xpu_runtime>();
  rt->device = device;
  XPU_HIP_RETURN(hipSetDevice(device));
  hipDeviceProp_t prop{};
  XPU_HIP_RETURN(hipGetDeviceProperties(&prop, device));
  rt->name = prop.name;
  if (rt->name.empty()) {
    char buf[256] = {0};
    if (hipDeviceGetName(buf, sizeof(buf), device) == hipSuccess) rt->name = buf;
  }
  if (rt->name.empty()) rt->name = "AMD Instinct (" + std::string(prop.gcnArchName) + ")";
  rt->arch = prop.gcnArchName;
  rt->total_memory = prop.totalGlobalMem;
  rt->compute_units = static_cast<uint32_t>(prop.multiProcessorCount);
  rt->max_shared = static_cast<uint32_t>(prop.sharedMemPerBlock);
  if (rt->arch.rfind("gfx950", 0) != 0)
    return set_error(XPU_ERR_DEVICE, "unsupported GPU '" + rt->name + "' (" + rt->arch +
                                         "): kernels are built for gfx950 (MI355X)");
  XPU_HIP_RETURN(hipStreamCreateWithFlags(&rt->stream, hipStreamNonBlocking));
  if (int rc = xpu::noalloc_scratch_setup(device)) return rc;

  std::string path;
  if (module_path && *module_path) path = module_path;
  else if (const char *env = std::getenv("XPU_KERNELS")) path = env;
  else path = xpu::library_directory() + "/xpu_kernels.hsaco";
  std::ifstream file(path, std::ios::binary | std::ios::ate);
  if (!file)
    return set_error(XPU_ERR_NOT_FOUND, "cannot open gfx950 kernel module " + path +
                                            "; build it with __graft_entry__.build()");
  const auto length = file.tellg();
  if (length <= 0) return set_error(XPU_ERR_NOT_FOUND, "empty kernel module: " + path);
  std::vector<char> image(static_cast<size_t>(length));
  file.seekg(0);
  if (!file.read(image.data(), length))
    return set_error(XPU_ERR_NOT_FOUND, "cannot read kernel module: " + path);
  XPU_HIP_RETURN(hipModuleLoadData(&rt->module, image.data()));
  for (const std::string &name : xpu::elf_kernel_names(image)) {
    xpu::KernelInfo k;
    k.name = name;
    XPU_HIP_RETURN(hipModuleGetFunction(&k.function, rt->module, name.c_str()));
    k.rule = xpu::find_rule(name);
    rt->kernels.push_back(std::move(k));
  }
  std::sort(rt->kernels.begin(), rt->kernels.end(),
            [](const xpu::KernelInfo &a, const xpu::KernelInfo &b) { return a.name < b.name; });
  if (rt->kernels.size() < 8)
    return set_error(XPU_ERR_NOT_FOUND, "kernel module " + path + " exposes " +
                                            std::to_string(rt->kernels.size()) +
                                            " kernels; at least 8 are required");
  rt->module_path = path;
  *out = rt.release();
  return XPU_OK;
}

void xpu_rt_destroy(xpu_runtime *rt) { delete rt; }

static int copy_string(const std::string &s, char *buf, size_t len) {
  if (!buf || len == 0) return set_error(XPU_ERR_INVALID, "null string buffer");
  std::snprintf(buf, len, "%s", s.c_str());
  return XPU_OK;
}

int xpu_rt_device_name(const xpu_runtime *rt, char *buf, size_t len) {
  if (!rt) return set_error(XPU_ERR_INVALID, "null runtime");
  return copy_string(rt->name, buf, len);
}

int xpu_rt_device_arch(const xpu_runtime *rt, char *buf, size_t len) {
  if (!rt) return set_error(XPU_ERR_INVALID, "null runtime");
  return copy_string(rt->arch, buf, len);
}

int xpu_rt_device_memory(const xpu_runtime *rt, uint64_t *bytes) {
  if (!rt || !bytes) return set_error(XPU_ERR_INVALID, "null argument");
  *bytes = rt->total_memory;
  return XPU_OK;
}

int xpu_rt_compute_units(const xpu_runtime *rt, uint32_t *count) {
  if (!rt || !count) return set_error(XPU_ERR_INVALID, "null argument");
  *count = rt->compute_units;
  return XPU_OK;
}

int xpu_rt_require_device_and_memory(const xpu_runtime *rt, uint64_t required_bytes) {
  if (!rt) return set_error(XPU_ERR_INVALID, "null runtime");
  XPU_HIP_RETURN(hipSetDevice(rt->device));
  size_t free_bytes = 0, total_bytes = 0;
  XPU_HIP_RETURN(hipMemGetInfo(&free_bytes, &total_bytes));
  constexpr uint64_t reserve = 512ull << 20;
  if (free_bytes < required_bytes || free_bytes - required_bytes < reserve)
    return set_error(XPU_ERR_DEVICE,
                     "insufficient device memory: need " +
                         std::to_string((required_bytes + (1ull << 20) - 1) >> 20) +
                         " MiB plus a 512 MiB reserve, " + std::to_string(free_bytes >> 20) +
                         " MiB free");
  return XPU_OK;
}

int xpu_rt_alloc(xpu_runtime *rt, uint64_t bytes, uint64_t alignment, void **out) {
  if (!rt || !out) return set_error(XPU_ERR_INVALID, "null argument");
  *out = nullptr;
  if (alignment == 0) alignment = 256;
  if ((alignment & (alignment - 1)) != 0 || alignment > 4096)
    return set_error(XPU_ERR_INVALID, "alignment must be a power of two <= 4096");
  XPU_HIP_RETURN(hipSetDevice(rt->device));
  void *p = nullptr;
  XPU_HIP_RETURN(hipMalloc(&p, bytes ? bytes : 1));
  if (reinterpret_cast<uintptr_t>(p) % alignment != 0) {
    (void)hipFree(p);
    return set_error(XPU_ERR_HIP, "hipMalloc returned memory below the requested alignment");
  }
  rt->allocations[p] = p;
  *out = p;
  return XPU_OK;
}

int xpu_rt_free(xpu_runtime *rt, void *ptr) {
  if (!rt) return set_error(XPU_ERR_INVALID, "null runtime");
  auto it = rt->allocations.find(ptr);
  if (it == rt->allocations.end())
    return set_error(XPU_ERR_INVALID, "pointer was not allocated by this runtime");
  XPU_HIP_RETURN(hipStreamSynchronize(rt->stream));
  XPU_HIP_RETURN(hipFree(it->second));
  rt->allocations.erase(it);
  return XPU_OK;
}

static int copy_sync(xpu_runtime *rt, void *dst, const void *src, size_t bytes, hipMemcpyKind kind) {
  if (!rt) return set_error(XPU_ERR_INVALID, "null runtime");
  if (bytes == 0) return XPU_OK;
  if (!dst || !src) return set_error(XPU_ERR_INVALID, "null copy pointer");
  XPU_HIP_RETURN(hipMemcpyAsync(dst, src, bytes, kind, rt->stream));
  XPU_HIP_RETURN(hipStreamSynchronize(rt->stream));
  return XPU_OK;
}

int xpu_rt_copy_to_device(xpu_runtime *rt, void *dst, const void *src, size_t bytes) {
  return copy_sync(rt, dst, src, bytes, hipMemcpyHostToDevice);
}
int xpu_rt_copy_from_device(xpu_runtime *rt, void *dst, const void *src, size_t bytes) {
  return copy_sync(rt, dst, src, bytes, hipMemcpyDeviceToHost);
}
int xpu_rt_copy_device(xpu_runtime *rt, void *dst, const void *src, size_t bytes) {
  return copy_sync(rt, dst, src, bytes, hipMemcpyDeviceToDevice);
}

int xpu_rt_memset(xpu_runtime *rt, void *dst, int value, size_t bytes) {
  if (!rt || !dst) return set_error(XPU_ERR_INVALID, "null argument");
  XPU_HIP_RETURN(hipMemsetAsync(dst, value, bytes, rt->stream));
  XPU_HIP_RETURN(hipStreamSynchronize(rt->stream));
  return XPU_OK;
}

int xpu_rt_launch(xpu_runtime *rt, const char *entry_fragment, uint32_t work_items,
                  const xpu_kernel_arg *args, uint32_t nargs) {
  if (!rt || !entry_fragment) return set_error(XPU_ERR_INVALID, "null argument");
  const xpu::KernelInfo *selected = nullptr;
  for (const auto &k : rt->kernels)
    if (k.name.find(entry_fragment) != std::string::npos) {
      if (selected)
        return set_error(XPU_ERR_INVALID, std::string("ambiguous kernel entry: ") + entry_fragment);
      selected = &k;
    }
  if (!selected)
    return set_error(XPU_ERR_NOT_FOUND,
                     std::string("kernel is absent from module: ") + entry_fragment);
  if (!selected->rule)
    return set_error(XPU_ERR_INVALID, "kernel " + selected->name +
                                          " has no work-item launch rule; use xpu_rt_launch_grid");
  const xpu::LaunchRule &rule = *selected->rule;
  const size_t want = std::strlen(rule.signature);
  if (nargs != want)
    return set_error(XPU_ERR_INVALID, selected->name + " takes " + std::to_string(want) +
                                          " arguments, got " + std::to_string(nargs));
  for (uint32_t i = 0; i < nargs; ++i) {
    const size_t size = (rule.signature[i] == 'p' || rule.signature[i] == 'q') ? 8 : 4;
    if (!args || args[i].size != size || !args[i].value)
      return set_error(XPU_ERR_INVALID, "argument " + std::to_string(i) + " (" +
                                            std::to_string(args ? args[i].size : 0) +
                                            " bytes) rejected for " + selected->name);
  }
  xpu::Geometry g{};
  int rc = rule.geometry(work_items, args, *rt, g);
  if (rc) return rc;
  if (g.grid == 0) return XPU_OK;
  XPU_HIP_RETURN(hipSetDevice(rt->device));
  rc = rt->launch(*selected, g.grid, 1, g.block, g.shared, args, nargs);
  if (rc) return rc;
  const hipError_t e = hipStreamSynchronize(rt->stream);
  if (e != hipSuccess) return set_error(XPU_ERR_HIP, xpu::hip_message(e, entry_fragment, __FILE__, __LINE__));
  return XPU_OK;
}

int xpu_rt_launch_grid(xpu_runtime *rt, const char *kernel_name, uint32_t grid_x, uint32_t grid_y,
                       uint32_t block_x, uint32_t shared_bytes, const xpu_kernel_arg *args,
                       uint32_t nargs) {
  if (!rt || !kernel_name) return set_error(XPU_ERR_INVALID, "null argument");
  const xpu::KernelInfo *k = rt->find_exact(kernel_name);
  if (!k) return set_error(XPU_ERR_NOT_FOUND, std::string("kernel is absent from module: ") + kernel_name);
  return rt->launch(*k, grid_x, grid_y, block_x, shared_bytes, args, nargs);
}

int xpu_module_kernel_names(const char *path, char *buf, size_t len) {
  if (!buf || len == 0) return set_error(XPU_ERR_INVALID, "null buffer");
  std::string p;
  if (path && *path) p = path;
  else p = xpu::library_directory() + "/xpu_kernels.hsaco";
  std::ifstream file(p, std::ios::binary | std::ios::ate);
  if (!file) return set_error(XPU_ERR_NOT_FOUND, "cannot open kernel module " + p);
  const auto length = file.tellg();
  std::vector<char> image(length > 0 ? static_cast<size_t>(length) : 0);
  file.seekg(0);
  if (image.empty() || !file.read(image.data(), length))
    return set_error(XPU_ERR_NOT_FOUND, "cannot read kernel module " + p);
  std::string joined;
  for (const std::string &name : xpu::elf_kernel_names(image)) joined += name + "\n";
  if (joined.size() + 1 > len) return set_error(XPU_ERR_INVALID, "buffer too small for kernel names");
  std::memcpy(buf, joined.c_str(), joined.size() + 1);
  return XPU_OK;
}

int xpu_rt_kernel_count(const xpu_runtime *rt, uint32_t *count) {
  if (!rt || !count) return set_error(XPU_ERR_INVALID, "null argument");
  *count = static_cast<uint32_t>(rt->kernels.size());
  return XPU_OK;
}

int xpu_rt_kernel_name(const xpu_runtime *rt, uint32_t index, char *buf, size_t len) {
  if (!rt) return set_error(XPU_ERR_INVALID, "null runtime");
  if (index >= rt->kernels.size()) return set_error(XPU_ERR_INVALID, "kernel index out of range");
  return copy_string(rt->kernels[index].name, buf, len);
}

int xpu_rt_module_global(xpu_runtime *rt, const char *name, void **dptr, uint64_t *bytes) {
  if (!rt || !name || !dptr || !bytes) return set_error(XPU_ERR_INVALID, "null argument");
  XPU_HIP_RETURN(hipSetDevice(rt->device));
  hipDeviceptr_t p = nullptr;
  size_t n = 0;
  if (hipModuleGetGlobal(&p, &n, rt->module, name) != hipSuccess || !p)
    return set_error(XPU_ERR_NOT_FOUND, std::string("code object has no global ") + name);
  *dptr = reinterpret_cast<void *>(p);
  *bytes = n;
  return XPU_OK;
}

int xpu_rt_synchronize(xpu_runtime *rt) {
  if (!rt) return set_error(XPU_ERR_INVALID, "null runtime");
  XPU_HIP_RETURN(hipStreamSynchronize(rt->stream));
  return XPU_OK;
}

void *xpu_rt_stream(xpu_runtime *rt) { return rt ? rt->stream : nullptr; }

int xpu_rt_event_create(xpu_runtime *rt, void **event) {
  if (!rt || !event) return set_error(XPU_ERR_INVALID, "null argument");
  hipEvent_t e = nullptr;
  XPU_HIP_RETURN(hipEventCreate(&e));
  *event = e;
  return XPU_OK;
}

int xpu_rt_event_record(xpu_runtime *rt, void *event) {
  if (!rt || !event) return set_error(XPU_ERR_INVALID, "null argument");
  XPU_HIP_RETURN(hipEventRecord(static_cast<hipEvent_t>(event), rt->stream));
  return XPU_OK;
}

int xpu_rt_event_elapsed_ms(void *start, void *stop, float *ms) {
  if (!start || !stop || !ms) return set_error(XPU_ERR_INVALID, "null argument");
  XPU_HIP_RETURN(hipEventSynchronize(static_cast<hipEvent_t>(stop)));
  XPU_HIP_RETURN(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)));
  return XPU_OK;
}

int xpu_rt_event_destroy(void *event) {
  if (!event) return XPU_OK;
  XPU_HIP_RETURN(hipEventDestroy(static_cast<hipEvent_t>(event)));
  return XPU_OK;
}

int xpu_rt_capture_begin(xpu_runtime *rt) {
  if (!rt) return set_error(XPU_ERR_INVALID, "null runtime");
  XPU_HIP_RETURN(hipStreamBeginCapture(rt->stream, hipStreamCaptureModeThreadLocal));
  return XPU_OK;
}

int xpu_rt_capture_end(xpu_runtime *rt, void **graph_exec) {
  if (!rt || !graph_exec) return set_error(XPU_ERR_INVALID, "null argument");
  hipGraph_t graph = nullptr;
  XPU_HIP_RETURN(hipStreamEndCapture(rt->stream, &graph));
  hipGraphExec_t exec = nullptr;
  const hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  if (e != hipSuccess) return set_error(XPU_ERR_HIP, xpu::hip_message(e, "hipGraphInstantiate", __FILE__, __LINE__));
  *graph_exec = exec;
  return XPU_OK;
}

int xpu_rt_graph_launch(xpu_runtime *rt, void *graph_exec) {
  if (!rt || !graph_exec) return set_error(XPU_ERR_INVALID, "null argument");
  XPU_HIP_RETURN(hipGraphLaunch(static_cast<hipGraphExec_t>(graph_exec), rt->stream));
  return XPU_OK;
}

int xpu_rt_graph_destroy(void *graph_exec) {
  if (!graph_exec) return XPU_OK;
  XPU_HIP_RETURN(hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph_exec)));
  return XPU_OK;
}

}  // extern "C"
