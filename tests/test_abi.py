"""The C-ABI library loads without a GPU and exports every function that
include/*.h declares; the code object holds the reference's kernel entries."""
import ctypes
import os
import re
import subprocess

import pytest

import xpu_playground_amd as xpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(REPO, "include")

# qwen3/kernels_entry.cpp:8-72
REFERENCE_ENTRIES = ["QwenEmbedding", "QwenRmsNorm", "QwenGemv", "QwenQkvRopeCache", "QwenAttention",
                     "QwenAdd", "QwenSiluMultiply", "QwenArgmax"]


def declared_functions():
    names = []
    for fn in sorted(os.listdir(INCLUDE)):
        if not fn.endswith(".h"):
            continue
        text = open(os.path.join(INCLUDE, fn)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b(\w+)\s*\([^;{]*\)\s*;", text, flags=re.M):
            names.append(m.group(1))
    return names


def test_headers_declare_the_boundary():
    names = declared_functions()
    required = ["xpu_rt_create", "xpu_rt_launch", "xpu_gemv", "xpu_gemm", "run_gemv", "run_gemm"]
    if os.path.exists(os.path.join(INCLUDE, "xpu_qwen3.h")):
        required += ["xpu_qwen3_create", "xpu_qwen3_decode", "xpu_qwen3_generate", "run_qwen3"]
    for required in required:
        assert required in names, required


def test_library_exports_every_declared_symbol():
    lib = xpu.library()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_code_object_contains_reference_entries_and_kernels():
    names = xpu.module_kernel_names()
    for entry in REFERENCE_ENTRIES:
        # the runtime's launch by fragment must resolve uniquely (level_zero_runtime.cpp:230-236)
        assert sum(entry in n for n in names) == 1, entry
    assert any(n.startswith("xpu_gemv_") for n in names)
    assert any(n.startswith("xpu_gemm_") for n in names)
    assert "xpu_q3_attention" in names


def test_runtime_errors_cross_the_abi_as_codes():
    lib = xpu.library()
    assert lib.xpu_rt_alloc(None, 16, 256, ctypes.byref(ctypes.c_void_p())) == 1
    assert b"null" in lib.xpu_last_error()
    assert lib.xpu_module_kernel_names(b"/nonexistent.hsaco", ctypes.create_string_buffer(16), 16) == 3


@pytest.mark.parametrize("program", ["gemv", "gemm", "qwen3_hip", "peak compute", "peak mem", "peak gemm"])
def test_cli_rejects_bad_flags_without_touching_a_gpu(program):
    program, *mode = program.split()
    exe = [os.path.join(xpu.BUILD_DIR, program)] + mode
    out = subprocess.run(exe + ["--bogus", "1"], capture_output=True, text=True, timeout=60)
    assert out.returncode == 1
    assert "unknown option" in out.stderr
    out = subprocess.run(exe + ["--help"], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0 and "Usage" in out.stdout


def test_peak_launcher_modes():
    exe = os.path.join(xpu.BUILD_DIR, "peak")
    out = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert out.returncode == 1 and "missing benchmark mode" in out.stderr
    # the reference's modes only (peak_sycl.cpp:47-50)
    for mode in ("flops", "sync"):
        out = subprocess.run([exe, mode], capture_output=True, text=True, timeout=60)
        assert out.returncode == 1 and "unknown benchmark mode" in out.stderr
    out = subprocess.run([exe, "--help"], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0 and "compute" in out.stdout and "mem" in out.stdout
