"""xpu_gemm_noalloc (include/xpu_kernels.h), the GEMM entry point that
allocates nothing: its padded operand copies go into a fixed per-GPU scratch
array. Called through the C ABI and checked bit for bit against xpu_gemm,
which runs the same kernels with the runtime's own workspace, on two calls in
a row (the second smaller, so stale scratch contents from the first would
show), plus the size limit and the in-place case."""
import ctypes

import numpy as np
import pytest

import oracle_lib as orc
import xpu_playground_amd as xpu

pytestmark = pytest.mark.gpu

LIMIT = 32 << 20  # XPU_GEMM_NOALLOC_SCRATCH_BYTES


def run_both(rt, a, b, m, n, k, dtype, offset_a=0):
    lib = xpu.library()
    da = rt.alloc(a.size * 2 + 16)
    db, dc1, dc2 = rt.upload(b), rt.alloc(m * n * 2), rt.alloc(m * n * 2)
    rt.copy_to(da + offset_a, a)
    try:
        for c in (dc1, dc2):
            rt.copy_to(c, np.full(m * n, 0x7FC0, np.uint16))  # NaN codes: every output must be written
        assert lib.xpu_gemm(rt.handle, dtype, ctypes.c_void_p(da + offset_a), ctypes.c_void_p(db),
                            ctypes.c_void_p(dc1), m, n, k) == 0, lib.xpu_last_error()
        assert lib.xpu_gemm_noalloc(rt.handle, dtype, ctypes.c_void_p(da + offset_a), ctypes.c_void_p(db),
                                    ctypes.c_void_p(dc2), m, n, k) == 0, lib.xpu_last_error()
        rt.synchronize()
        return rt.download(dc1, m * n, np.uint16), rt.download(dc2, m * n, np.uint16)
    finally:
        for p in (da, db, dc1, dc2):
            rt.free(p)


def test_noalloc_matches_xpu_gemm_on_consecutive_calls(rt):
    # first: the ragged BASELINE shape (both operands padded: 29.1 MB of the
    # 32 MiB array); second: a smaller ragged product that reuses the array
    cases = [(3000, 4097, 2050, xpu.FP16, 0), (300, 201, 130, xpu.BF16, 2), (64, 40, 24, xpu.BF16, 0)]
    for m, n, k, dtype, off in cases:
        print(f"noalloc gemm {m}x{n}x{k} dtype={dtype} A offset {off}", flush=True)
        a = orc.uniform(m * k, 31 + m, dtype)
        b = orc.uniform(k * n, 41 + n, dtype)
        ref, got = run_both(rt, a, b, m, n, k, dtype, off)
        assert np.array_equal(ref, got)
        if m * n <= 300 * 201:  # the oracle's bound on a small case
            exact = orc.gemm_f64(a, b, m, n, k, dtype)
            r = orc.decode(orc.encode(exact.astype(np.float32), dtype), dtype).astype(np.float64)
            g = orc.decode(got, dtype).astype(np.float64).reshape(m, n)
            assert np.linalg.norm(g - r) / np.linalg.norm(r) <= 1e-3


def test_noalloc_in_place_operands_need_no_scratch(rt):
    m = n = k = 512
    a = orc.uniform(m * k, 5, xpu.BF16)
    b = orc.uniform(k * n, 6, xpu.BF16)
    ref, got = run_both(rt, a, b, m, n, k, xpu.BF16)
    assert np.array_equal(ref, got)


def test_noalloc_rejects_needs_above_the_array(rt):
    # K = 4100 (not a multiple of 8): A is copied, 4096 x 4104 x 2 = 33.6 MB > 32 MiB
    lib = xpu.library()
    m, n, k = 4096, 64, 4100
    da, db, dc = rt.alloc(m * k * 2), rt.alloc(k * n * 2), rt.alloc(m * n * 2)
    try:
        rc = lib.xpu_gemm_noalloc(rt.handle, xpu.BF16, ctypes.c_void_p(da), ctypes.c_void_p(db),
                                  ctypes.c_void_p(dc), m, n, k)
        assert rc == 1
        assert b"scratch array" in lib.xpu_last_error()
    finally:
        for p in (da, db, dc):
            rt.free(p)
