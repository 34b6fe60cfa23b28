"""xpu_gemm_noalloc (include/xpu_kernels.h), the GEMM entry point that
allocates nothing: where xpu_gemm splits K, its FP32 partials go into a fixed
per-GPU scratch array instead of the runtime's workspace. Called through the
C ABI and checked bit for bit against xpu_gemm, which runs the same kernels
with the runtime's own workspace, on two split-K calls in a row (the second
smaller, so stale partials from the first would show), plus a shape that
needs no scratch and the size limit."""
import ctypes

import numpy as np
import pytest

import oracle_lib as orc
import xpu_playground_amd as xpu

pytestmark = pytest.mark.gpu

LIMIT = 16 << 20  # XPU_GEMM_NOALLOC_SCRATCH_BYTES


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


def split_bytes(rt, m, n, k):
    """The partials xpu_gemm keeps for this shape (gemm_api.cpp's rule), 0
    when it does not split K."""
    rows, cols = ctypes.c_uint32(), ctypes.c_uint32()
    assert xpu.library().xpu_gemm_tile(rt.handle, m, n, ctypes.byref(rows), ctypes.byref(cols)) == 0
    t128 = ((m + 127) // 128) * ((n + 127) // 128)
    nslices = (k + 63) // 64
    if (rows.value, cols.value) != (128, 128) or t128 * 2 > rt.compute_units or nslices < 8:
        return 0
    want = (rt.compute_units + t128 - 1) // t128
    spl = ((nslices + want - 1) // want + 1) // 2 * 2
    splits = (nslices + spl - 1) // spl
    nbytes = splits * m * ((n + 3) // 4 * 4) * 4
    return nbytes if splits >= 2 and (nslices >= 24 or nbytes <= 4 << 20) else 0


def test_noalloc_matches_xpu_gemm_on_consecutive_calls(rt):
    # first: 1024 x 1024 x 4096 bf16, 4 splits of 4 MiB (the whole array);
    # then smaller split-K products with ragged N and K and an offset A,
    # which reuse the array
    cases = [(1024, 1024, 4096, xpu.BF16, 0), (300, 201, 1030, xpu.FP16, 2), (64, 40, 520, xpu.BF16, 0)]
    for m, n, k, dtype, off in cases:
        need = split_bytes(rt, m, n, k)
        print(f"noalloc gemm {m}x{n}x{k} dtype={dtype} A offset {off}: {need} bytes of partials", flush=True)
        assert 0 < need <= LIMIT
        a = orc.uniform(m * k, 31 + m, dtype)
        b = orc.uniform(k * n, 41 + n, dtype)
        ref, got = run_both(rt, a, b, m, n, k, dtype, off)
        assert np.array_equal(ref, got)
        if m * n <= 300 * 201:  # the oracle's bound on a small case
            exact = orc.gemm_f64(a, b, m, n, k, dtype)
            r = orc.decode(orc.encode(exact.astype(np.float32), dtype), dtype).astype(np.float64)
            g = orc.decode(got, dtype).astype(np.float64).reshape(m, n)
            assert np.linalg.norm(g - r) / np.linalg.norm(r) <= 1e-3


def test_noalloc_without_split_needs_no_scratch(rt):
    m, n, k = 512, 512, 256  # 4 K-slices: no split
    assert split_bytes(rt, m, n, k) == 0
    a = orc.uniform(m * k, 5, xpu.BF16)
    b = orc.uniform(k * n, 6, xpu.BF16)
    ref, got = run_both(rt, a, b, m, n, k, xpu.BF16)
    assert np.array_equal(ref, got)


def test_noalloc_rejects_needs_above_the_array(rt):
    # 1280 x 1280 x 2048: 100 tiles of 128 x 128, 3 splits of 6.5 MB > 16 MiB
    lib = xpu.library()
    m, n, k = 1280, 1280, 2048
    need = split_bytes(rt, m, n, k)
    print(f"noalloc gemm {m}x{n}x{k}: {need} bytes of partials", flush=True)
    assert need > LIMIT
    da, db, dc = rt.alloc(m * k * 2), rt.alloc(k * n * 2), rt.alloc(m * n * 2)
    try:
        rc = lib.xpu_gemm_noalloc(rt.handle, xpu.BF16, ctypes.c_void_p(da), ctypes.c_void_p(db),
                                  ctypes.c_void_p(dc), m, n, k)
        assert rc == 1
        assert b"scratch array" in lib.xpu_last_error()
    finally:
        for p in (da, db, dc):
            rt.free(p)
