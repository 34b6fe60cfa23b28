/*
 * xpu_runtime.h - thin C-ABI HIP runtime for gfx950 (MI355X).
 *
 * Replaces qwen3::LevelZeroRuntime (reference qwen3/level_zero_runtime.hpp:18-48,
 * qwen3/level_zero_runtime.cpp:52-255) and the Level Zero runtime class of
 * level_zero/peak_l0.cpp:101-360. One runtime owns one HIP device, one HIP
 * stream (default priority), the kernel code object (hipModuleLoad) and every
 * device allocation it made (all freed by xpu_rt_destroy, like the
 * reference's destructor, level_zero_runtime.cpp:163-175).
 *
 * Conventions: every function returns 0 on success and a nonzero code on
 * failure; xpu_last_error() then describes the failure (thread-local). No C++
 * exception crosses this boundary. Pointers to device memory are plain
 * void*; sizes are bytes unless stated. Not thread-safe per runtime (same as
 * the reference: one immediate command list, no locks).
 */
#ifndef XPU_RUNTIME_H
#define XPU_RUNTIME_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define XPU_OK 0
#define XPU_ERR_INVALID 1     /* bad argument (shape, pointer, option) */
#define XPU_ERR_HIP 2         /* a HIP call failed */
#define XPU_ERR_NOT_FOUND 3   /* kernel / file absent */
#define XPU_ERR_DEVICE 4      /* no gfx950 device or not enough memory */
#define XPU_ERR_VERIFY 5      /* verification failed (apps) */

typedef struct xpu_runtime xpu_runtime;

/* One kernel argument: size in bytes and a pointer to its value
 * (reference qwen3/level_zero_runtime.hpp:13-16, kernel_argument :50-52). */
typedef struct {
  size_t size;
  const void *value;
} xpu_kernel_arg;

/* Last error message of the calling thread ("" when none). */
const char *xpu_last_error(void);

/* Create a runtime on HIP device `device` (-1: $XPU_DEVICE or 0) loading the
 * code object at module_path (NULL: xpu_kernels.hsaco next to this library,
 * or $XPU_KERNELS). Replaces LevelZeroRuntime(module_path)
 * (level_zero_runtime.cpp:52-161). Fails with XPU_ERR_DEVICE unless the
 * device is gfx950. */
int xpu_rt_create(const char *module_path, int device, xpu_runtime **out);
void xpu_rt_destroy(xpu_runtime *rt);

/* Device name / gcnArchName / total memory / compute units
 * (level_zero_runtime.hpp:32-33). */
int xpu_rt_device_name(const xpu_runtime *rt, char *buf, size_t len);
int xpu_rt_device_arch(const xpu_runtime *rt, char *buf, size_t len);
int xpu_rt_device_memory(const xpu_runtime *rt, uint64_t *bytes);
int xpu_rt_compute_units(const xpu_runtime *rt, uint32_t *count);

/* gfx950 check plus required_bytes + 512 MiB reserve against free memory
 * (replaces require_bmg_and_memory, level_zero_runtime.cpp:177-195). */
int xpu_rt_require_device_and_memory(const xpu_runtime *rt, uint64_t required_bytes);

/* Device allocation owned by the runtime (allocate_device,
 * level_zero_runtime.cpp:197-210); alignment must be a power of two <= 4096
 * (hipMalloc returns 4096-aligned blocks for these sizes). */
int xpu_rt_alloc(xpu_runtime *rt, uint64_t bytes, uint64_t alignment, void **out);
int xpu_rt_free(xpu_runtime *rt, void *ptr);

/* Synchronous copies (copy_to_device / copy_from_device,
 * level_zero_runtime.cpp:212-223) and a device-to-device copy. */
int xpu_rt_copy_to_device(xpu_runtime *rt, void *dst, const void *src, size_t bytes);
int xpu_rt_copy_from_device(xpu_runtime *rt, void *dst, const void *src, size_t bytes);
int xpu_rt_copy_device(xpu_runtime *rt, void *dst, const void *src, size_t bytes);
/* Fill with a byte value (not for use under graph capture). */
int xpu_rt_memset(xpu_runtime *rt, void *dst, int value, size_t bytes);

/* Blocking launch by entry-name fragment with the reference's work-item
 * convention (level_zero_runtime.cpp:225-255): the unique kernel whose name
 * contains `entry_fragment` (ambiguity is an error) is launched with the
 * geometry its table entry derives from work_items, then the stream is
 * synchronised. */
int xpu_rt_launch(xpu_runtime *rt, const char *entry_fragment, uint32_t work_items,
                  const xpu_kernel_arg *args, uint32_t nargs);

/* Asynchronous launch of an exact kernel name with explicit geometry on the
 * runtime's stream. */
int xpu_rt_launch_grid(xpu_runtime *rt, const char *kernel_name, uint32_t grid_x,
                       uint32_t grid_y, uint32_t block_x, uint32_t shared_bytes,
                       const xpu_kernel_arg *args, uint32_t nargs);

/* Newline-separated kernel names of a code object file (NULL: the default
 * module next to this library); needs no GPU. */
int xpu_module_kernel_names(const char *path, char *buf, size_t len);

/* Number and names of the kernels in the loaded code object. */
int xpu_rt_kernel_count(const xpu_runtime *rt, uint32_t *count);
int xpu_rt_kernel_name(const xpu_runtime *rt, uint32_t index, char *buf, size_t len);

/* Device address and size of a global variable of the loaded code object
 * (hipModuleGetGlobal), e.g. the timestamp rings of the XPU_STAMPS build;
 * XPU_ERR_NOT_FOUND when the module has no such symbol. No reference
 * counterpart (a profiling aid). */
int xpu_rt_module_global(xpu_runtime *rt, const char *name, void **dptr, uint64_t *bytes);

int xpu_rt_synchronize(xpu_runtime *rt);
/* The runtime's hipStream_t, as an opaque pointer. */
void *xpu_rt_stream(xpu_runtime *rt);

/* Events on the runtime's stream (hipEventRecord / hipEventElapsedTime). */
int xpu_rt_event_create(xpu_runtime *rt, void **event);
int xpu_rt_event_record(xpu_runtime *rt, void *event);
int xpu_rt_event_elapsed_ms(void *start, void *stop, float *ms);
int xpu_rt_event_destroy(void *event);

/* Stream capture of the runtime's stream into an executable HIP graph. */
int xpu_rt_capture_begin(xpu_runtime *rt);
int xpu_rt_capture_end(xpu_runtime *rt, void **graph_exec);
int xpu_rt_graph_launch(xpu_runtime *rt, void *graph_exec);
int xpu_rt_graph_destroy(void *graph_exec);

#ifdef __cplusplus
}
#endif
#endif
