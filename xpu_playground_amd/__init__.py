"""ctypes bindings to the gfx950 hot-path library (build/libxpu_playground.so).

The C ABI is declared in include/xpu_runtime.h, include/xpu_kernels.h and
include/xpu_qwen3.h. Every compute call runs the HIP kernels of
build/xpu_kernels.hsaco; there is no CPU fallback: if the library or the code
object is missing, or no gfx950 device is visible, the calls raise.
"""
from __future__ import annotations

import ctypes
import os
import weakref
from ctypes import POINTER, c_char_p, c_double, c_float, c_int, c_size_t, c_uint32, c_uint64, c_void_p

PACKAGE_DIR = os.path.dirname(os.path.abspath(__file__))
BUILD_DIR = os.path.join(PACKAGE_DIR, "build")
LIBRARY_PATH = os.path.join(BUILD_DIR, "libxpu_playground.so")
MODULE_PATH = os.path.join(BUILD_DIR, "xpu_kernels.hsaco")

BF16 = 0
FP16 = 1

XPU_OK = 0


class XpuError(RuntimeError):
    """A C-ABI call returned a nonzero status."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[xpu error {code}] {message}")
        self.code = code


class KernelArg(ctypes.Structure):
    _fields_ = [("size", c_size_t), ("value", c_void_p)]


class Qwen3Config(ctypes.Structure):
    """xpu_qwen3_config (include/xpu_qwen3.h)."""

    _fields_ = [
        ("hidden", c_uint32),
        ("intermediate", c_uint32),
        ("layers", c_uint32),
        ("heads", c_uint32),
        ("kv_heads", c_uint32),
        ("head_dim", c_uint32),
        ("vocab", c_uint32),
        ("rms_eps", c_float),
        ("rope_theta", c_double),
        ("tied", c_uint32),
    ]


_lib = None


def _declare(lib):
    sig = {
        "xpu_last_error": (c_char_p, []),
        "xpu_rt_create": (c_int, [c_char_p, c_int, POINTER(c_void_p)]),
        "xpu_rt_destroy": (None, [c_void_p]),
        "xpu_rt_device_name": (c_int, [c_void_p, c_char_p, c_size_t]),
        "xpu_rt_device_arch": (c_int, [c_void_p, c_char_p, c_size_t]),
        "xpu_rt_device_memory": (c_int, [c_void_p, POINTER(c_uint64)]),
        "xpu_rt_compute_units": (c_int, [c_void_p, POINTER(c_uint32)]),
        "xpu_rt_require_device_and_memory": (c_int, [c_void_p, c_uint64]),
        "xpu_rt_alloc": (c_int, [c_void_p, c_uint64, c_uint64, POINTER(c_void_p)]),
        "xpu_rt_free": (c_int, [c_void_p, c_void_p]),
        "xpu_rt_copy_to_device": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t]),
        "xpu_rt_copy_from_device": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t]),
        "xpu_rt_copy_device": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t]),
        "xpu_rt_memset": (c_int, [c_void_p, c_void_p, c_int, c_size_t]),
        "xpu_rt_launch": (c_int, [c_void_p, c_char_p, c_uint32, POINTER(KernelArg), c_uint32]),
        "xpu_rt_launch_grid": (
            c_int,
            [c_void_p, c_char_p, c_uint32, c_uint32, c_uint32, c_uint32, POINTER(KernelArg), c_uint32],
        ),
        "xpu_module_kernel_names": (c_int, [c_char_p, c_char_p, c_size_t]),
        "xpu_rt_kernel_count": (c_int, [c_void_p, POINTER(c_uint32)]),
        "xpu_rt_module_global": (c_int, [c_void_p, c_char_p, POINTER(c_void_p), POINTER(c_uint64)]),
        "xpu_rt_kernel_name": (c_int, [c_void_p, c_uint32, c_char_p, c_size_t]),
        "xpu_rt_synchronize": (c_int, [c_void_p]),
        "xpu_rt_stream": (c_void_p, [c_void_p]),
        "xpu_rt_event_create": (c_int, [c_void_p, POINTER(c_void_p)]),
        "xpu_rt_event_record": (c_int, [c_void_p, c_void_p]),
        "xpu_rt_event_elapsed_ms": (c_int, [c_void_p, c_void_p, POINTER(c_float)]),
        "xpu_rt_event_destroy": (c_int, [c_void_p]),
        "xpu_rt_capture_begin": (c_int, [c_void_p]),
        "xpu_rt_capture_end": (c_int, [c_void_p, POINTER(c_void_p)]),
        "xpu_rt_graph_launch": (c_int, [c_void_p, c_void_p]),
        "xpu_rt_graph_destroy": (c_int, [c_void_p]),
        "xpu_gemv": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint64]),
        "xpu_fill_uniform": (c_int, [c_void_p, c_int, c_void_p, c_uint64, c_uint64]),
        "xpu_fill_reference_gemv": (
            c_int,
            [c_void_p, c_int, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32],
        ),
    }
    optional = {
        "xpu_gemm": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32]),
        "xpu_gemm_noalloc": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32]),
        "xpu_gemm_tile": (c_int, [c_void_p, c_uint32, c_uint32, POINTER(c_uint32), POINTER(c_uint32)]),
        "xpu_qwen3_preset": (c_int, [c_char_p, POINTER(Qwen3Config)]),
        "xpu_qwen3_fill_tensor": (
            c_int,
            [POINTER(Qwen3Config), c_uint64, c_float, c_int, c_uint32, c_void_p, c_uint64],
        ),
        "xpu_qwen3_rope_tables": (c_int, [c_void_p, c_void_p, c_uint32, c_uint32, c_double]),
        "xpu_qwen3_create": (
            c_int,
            [c_void_p, POINTER(Qwen3Config), c_uint32, c_uint64, c_float, POINTER(c_void_p)],
        ),
        "xpu_qwen3_destroy": (None, [c_void_p]),
        "xpu_qwen3_set_mode": (c_int, [c_void_p, c_int]),
        "xpu_qwen3_set_prefill": (c_int, [c_void_p, c_int]),
        "xpu_qwen3_set_attention_split": (c_int, [c_void_p, c_uint32]),
        "xpu_qwen3_decode": (c_int, [c_void_p, c_uint32, c_uint32, POINTER(c_uint32)]),
        "xpu_qwen3_logits": (c_int, [c_void_p, c_void_p, c_uint64]),
        "xpu_qwen3_hidden": (c_int, [c_void_p, c_void_p, c_uint64]),
        "xpu_qwen3_generate": (
            c_int,
            [
                c_void_p,
                POINTER(c_uint32),
                c_uint32,
                c_uint32,
                c_int,
                POINTER(c_uint32),
                POINTER(c_uint32),
                POINTER(c_double),
                POINTER(c_double),
            ],
        ),
        "xpu_qwen3_read_config": (c_int, [c_char_p, POINTER(Qwen3Config)]),
        "xpu_qwen3_validate_checkpoint": (c_int, [c_char_p, POINTER(Qwen3Config)]),
        "xpu_qwen3_get_config": (c_int, [c_void_p, POINTER(Qwen3Config)]),
        "xpu_qwen3_create_from_checkpoint": (c_int, [c_void_p, c_char_p, c_uint32, POINTER(c_void_p)]),
        "xpu_synth_tokens": (c_int, [c_void_p, c_uint64, c_uint64, c_uint32]),
        "run_gemv": (c_int, [c_int, POINTER(c_char_p)]),
        "run_gemm": (c_int, [c_int, POINTER(c_char_p)]),
        "xpu_peak_mfma": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32]),
        "xpu_peak_read": (c_int, [c_void_p, c_void_p, c_uint64, c_void_p, c_uint32]),
        "run_peak_compute": (c_int, [c_int, POINTER(c_char_p)]),
        "run_peak_mem": (c_int, [c_int, POINTER(c_char_p)]),
        "run_qwen3": (c_int, [c_int, POINTER(c_char_p)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    for name, (res, args) in optional.items():
        fn = getattr(lib, name, None)
        if fn is not None:
            fn.restype = res
            fn.argtypes = args
    return lib


def library():
    """Load build/libxpu_playground.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIBRARY_PATH):
            raise RuntimeError(
                f"{LIBRARY_PATH} is missing: run __graft_entry__.build() (the HIP path has no fallback)"
            )
        _lib = _declare(ctypes.CDLL(LIBRARY_PATH))
    return _lib


def check(code: int) -> None:
    if code != XPU_OK:
        raise XpuError(code, library().xpu_last_error().decode(errors="replace"))


def module_kernel_names(path: str | None = None) -> list[str]:
    buf = ctypes.create_string_buffer(1 << 16)
    check(library().xpu_module_kernel_names(path.encode() if path else None, buf, len(buf)))
    return buf.value.decode().split()


class Args:
    """Builds an xpu_kernel_arg array and keeps the argument values alive."""

    def __init__(self):
        self._values = []
        self._sizes = []

    def ptr(self, p):
        self._values.append(c_void_p(p if isinstance(p, int) or p is None else p.value))
        self._sizes.append(8)
        return self

    def u32(self, v):
        self._values.append(c_uint32(v))
        self._sizes.append(4)
        return self

    def u64(self, v):
        self._values.append(c_uint64(v))
        self._sizes.append(8)
        return self

    def f32(self, v):
        self._values.append(c_float(v))
        self._sizes.append(4)
        return self

    def array(self):
        arr = (KernelArg * len(self._values))()
        for i, (v, s) in enumerate(zip(self._values, self._sizes)):
            arr[i].size = s
            arr[i].value = ctypes.cast(ctypes.pointer(v), c_void_p)
        return arr, len(self._values)


class Runtime:
    """Owner of one gfx950 device, stream, code object and allocations."""

    def __init__(self, module_path: str | None = None, device: int = -1):
        self.lib = library()
        self._dependents = weakref.WeakSet()
        handle = c_void_p()
        check(self.lib.xpu_rt_create(module_path.encode() if module_path else None, device, ctypes.byref(handle)))
        self.handle = handle

    def add_dependent(self, obj) -> None:
        """Register an object holding allocations of this runtime (an engine);
        close() closes it first, so it never frees through a destroyed
        runtime."""
        self._dependents.add(obj)

    def close(self):
        if self.handle:
            for dep in list(self._dependents):
                dep.close()
            self.lib.xpu_rt_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _string(self, fn):
        buf = ctypes.create_string_buffer(256)
        check(fn(self.handle, buf, len(buf)))
        return buf.value.decode()

    @property
    def device_name(self) -> str:
        return self._string(self.lib.xpu_rt_device_name)

    @property
    def arch(self) -> str:
        return self._string(self.lib.xpu_rt_device_arch)

    @property
    def compute_units(self) -> int:
        v = c_uint32()
        check(self.lib.xpu_rt_compute_units(self.handle, ctypes.byref(v)))
        return v.value

    @property
    def device_memory(self) -> int:
        v = c_uint64()
        check(self.lib.xpu_rt_device_memory(self.handle, ctypes.byref(v)))
        return v.value

    def kernel_names(self) -> list[str]:
        n = c_uint32()
        check(self.lib.xpu_rt_kernel_count(self.handle, ctypes.byref(n)))
        out = []
        for i in range(n.value):
            buf = ctypes.create_string_buffer(256)
            check(self.lib.xpu_rt_kernel_name(self.handle, i, buf, len(buf)))
            out.append(buf.value.decode())
        return out

    def alloc(self, nbytes: int, alignment: int = 256) -> int:
        p = c_void_p()
        check(self.lib.xpu_rt_alloc(self.handle, nbytes, alignment, ctypes.byref(p)))
        return p.value

    def free(self, ptr: int) -> None:
        check(self.lib.xpu_rt_free(self.handle, c_void_p(ptr)))

    def upload(self, array) -> int:
        """Allocate device memory and copy a contiguous numpy array into it."""
        import numpy as np

        a = np.ascontiguousarray(array)
        ptr = self.alloc(max(a.nbytes, 1))
        check(self.lib.xpu_rt_copy_to_device(self.handle, c_void_p(ptr), a.ctypes.data_as(c_void_p), a.nbytes))
        return ptr

    def copy_to(self, ptr: int, array) -> None:
        import numpy as np

        a = np.ascontiguousarray(array)
        check(self.lib.xpu_rt_copy_to_device(self.handle, c_void_p(ptr), a.ctypes.data_as(c_void_p), a.nbytes))

    def download(self, ptr: int, count: int, dtype) -> "np.ndarray":  # noqa: F821
        import numpy as np

        out = np.empty(count, dtype=dtype)
        check(self.lib.xpu_rt_copy_from_device(self.handle, out.ctypes.data_as(c_void_p), c_void_p(ptr), out.nbytes))
        return out

    def memset(self, ptr: int, value: int, nbytes: int) -> None:
        check(self.lib.xpu_rt_memset(self.handle, c_void_p(ptr), value, nbytes))

    def synchronize(self) -> None:
        check(self.lib.xpu_rt_synchronize(self.handle))

    def launch(self, fragment: str, work_items: int, args: Args) -> None:
        """Blocking launch with the reference's work-item convention."""
        arr, n = args.array()
        check(self.lib.xpu_rt_launch(self.handle, fragment.encode(), work_items, arr, n))

    def launch_grid(self, name: str, grid: int, block: int, shared: int, args: Args, grid_y: int = 1) -> None:
        arr, n = args.array()
        check(self.lib.xpu_rt_launch_grid(self.handle, name.encode(), grid, grid_y, block, shared, arr, n))

    def event(self) -> "Event":
        return Event(self)

    # ---- hot-path entry points
    def gemv(self, dtype: int, a: int, x: int, y: int, m: int, k: int, lda: int | None = None) -> None:
        check(self.lib.xpu_gemv(self.handle, dtype, c_void_p(a), c_void_p(x), c_void_p(y), m, k, lda or k))

    def gemm(self, dtype: int, a: int, b: int, c: int, m: int, n: int, k: int) -> None:
        check(self.lib.xpu_gemm(self.handle, dtype, c_void_p(a), c_void_p(b), c_void_p(c), m, n, k))

    def gemm_tile(self, m: int, n: int) -> tuple[int, int]:
        """The block tile (rows, cols) that gemm() uses for an m x n output."""
        rows, cols = ctypes.c_uint32(), ctypes.c_uint32()
        check(self.lib.xpu_gemm_tile(self.handle, m, n, ctypes.byref(rows), ctypes.byref(cols)))
        return rows.value, cols.value

    def fill_uniform(self, dtype: int, ptr: int, count: int, seed: int) -> None:
        check(self.lib.xpu_fill_uniform(self.handle, dtype, c_void_p(ptr), count, seed))

    def fill_reference_gemv(self, dtype: int, matrix: int, vector: int, m: int, k: int, ld: int) -> None:
        check(self.lib.xpu_fill_reference_gemv(self.handle, dtype, c_void_p(matrix), c_void_p(vector), m, k, ld))


class Event:
    def __init__(self, rt: Runtime):
        self.rt = rt
        self.handle = c_void_p()
        check(rt.lib.xpu_rt_event_create(rt.handle, ctypes.byref(self.handle)))

    def record(self) -> None:
        check(self.rt.lib.xpu_rt_event_record(self.rt.handle, self.handle))

    def elapsed_ms(self, stop: "Event") -> float:
        ms = c_float()
        check(self.rt.lib.xpu_rt_event_elapsed_ms(self.handle, stop.handle, ctypes.byref(ms)))
        return ms.value

    def __del__(self):
        try:
            if self.handle:
                self.rt.lib.xpu_rt_event_destroy(self.handle)
        except Exception:
            pass
