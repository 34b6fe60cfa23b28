"""GEMM on gfx950 MFMA vs the CPU oracle (FP64 accumulation, rounded to the
output type): rel-L2 <= 1e-3 and |error| <= 2 output ulps + gamma_K sum|a b|
elementwise; plus the reference's constant known-answer check."""
import numpy as np
import pytest

import oracle_lib as orc
import xpu_playground_amd as xpu

pytestmark = pytest.mark.gpu


def gpu_gemm(rt, a, b, m, n, k, dtype):
    da, db, dc = rt.upload(a), rt.upload(b), rt.alloc(m * n * 2)
    try:
        rt.gemm(dtype, da, db, dc, m, n, k)
        rt.synchronize()
        return rt.download(dc, m * n, np.uint16).reshape(m, n)
    finally:
        for p in (da, db, dc):
            rt.free(p)


def check(c, a, b, m, n, k, dtype, rows=None):
    exact = orc.gemm_f64(a, b, m, n, k, dtype, rows)
    got = orc.decode(c if rows is None else c[rows], dtype).astype(np.float64)
    ref = orc.decode(orc.encode(exact.astype(np.float32), dtype), dtype).astype(np.float64)
    rel = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-300)
    assert rel <= 1e-3, rel
    fa = np.abs(orc.decode(a, dtype).reshape(m, k).astype(np.float64))
    fb = np.abs(orc.decode(b, dtype).reshape(k, n).astype(np.float64))
    absab = (fa if rows is None else fa[rows]) @ fb
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(ref), 1e-30))) - (7 if dtype == 0 else 10))
    gamma = k * 2.0**-24 / (1 - k * 2.0**-24)
    bad = np.abs(got - ref) > 2 * ulp + gamma * absab
    assert not bad.any(), (int(bad.sum()), np.argwhere(bad)[:5])
    return rel


@pytest.mark.parametrize("dtype", [xpu.BF16, xpu.FP16])
@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (37, 53, 70), (256, 256, 64), (255, 257, 65), (300, 8, 16),
                                   (33, 17, 9), (512, 512, 1024), (1000, 600, 520)])
def test_gemm_small_shapes(rt, dtype, m, n, k):
    print(f"gemm dtype={dtype} {m}x{n}x{k}", flush=True)
    a = orc.uniform(m * k, 10 + m, dtype)
    b = orc.uniform(k * n, 20 + n, dtype)
    check(gpu_gemm(rt, a, b, m, n, k, dtype), a, b, m, n, k, dtype)


@pytest.mark.parametrize("dtype", [xpu.BF16, xpu.FP16])
@pytest.mark.parametrize("m,n,k", [(256, 256, 64), (255, 257, 65), (64, 40, 24)])
def test_gemm_pointers_two_bytes_past_alignment(rt, dtype, m, n, k):
    # A, B and C start 2 bytes past a 16-byte boundary: both operands are
    # staged from 2-byte aligned rows in place, and every C row starts 2 bytes
    # past a dword (or a 16-byte) boundary, the unaligned-C epilogue's cases.
    # Guard codes around C catch any store outside it.
    print(f"gemm unaligned pointers dtype={dtype} {m}x{n}x{k}", flush=True)
    a = orc.uniform(m * k, 30 + m, dtype)
    b = orc.uniform(k * n, 40 + n, dtype)
    guard = 0x7E7E
    pa, pb, pc = rt.alloc(m * k * 2 + 64), rt.alloc(k * n * 2 + 64), rt.alloc(m * n * 2 + 64)
    try:
        rt.copy_to(pc, np.full((m * n * 2 + 64) // 2, guard, np.uint16))
        rt.copy_to(pa + 2, a)
        rt.copy_to(pb + 2, b)
        rt.gemm(dtype, pa + 2, pb + 2, pc + 2, m, n, k)
        rt.synchronize()
        out = rt.download(pc, (m * n * 2 + 64) // 2, np.uint16)
    finally:
        for p in (pa, pb, pc):
            rt.free(p)
    assert out[0] == guard and np.all(out[1 + m * n:] == guard)
    check(out[1:1 + m * n].reshape(m, n), a, b, m, n, k, dtype)


def test_gemm_constant_known_answer(rt):
    # gemm.cpp:81-85,109-117 (and level_zero/peak_l0.cpp:910-917,936-943)
    for dtype, (m, n, k) in [(0, (4096, 4096, 4096)), (1, (3000, 4097, 2050))]:
        a = orc.encode(np.full(m * k, 0.5, np.float32), dtype)
        b = orc.encode(np.full(k * n, 0.25, np.float32), dtype)
        c = gpu_gemm(rt, a, b, m, n, k, dtype)
        assert np.all(orc.decode(c, dtype) == np.float32(orc.decode(orc.encode(np.array([0.125 * k], np.float32), dtype), dtype)[0]))


def test_gemm_m1_bf16_4096(rt):
    # bf16 4096^3, seeded U[-1,1]; FP64 on 256 sampled rows
    # plus a column-checksum over all rows
    m = n = k = 4096
    da, db, dc = rt.alloc(m * k * 2), rt.alloc(k * n * 2), rt.alloc(m * n * 2)
    rt.fill_uniform(0, da, m * k, 5)
    rt.fill_uniform(0, db, k * n, 6)
    rt.gemm(0, da, db, dc, m, n, k)
    rt.synchronize()
    a, b = rt.download(da, m * k, np.uint16), rt.download(db, k * n, np.uint16)
    c = rt.download(dc, m * n, np.uint16).reshape(m, n)
    rows = np.sort(np.random.default_rng(0).choice(m, 256, replace=False))
    print("rel-L2", check(c, a, b, m, n, k, 0, rows))
    fa = orc.decode(a, 0).reshape(m, k).astype(np.float64)
    fb = orc.decode(b, 0).reshape(k, n).astype(np.float64)
    colsum_exact = fa.sum(axis=0) @ fb
    fc = orc.decode(c, 0).astype(np.float64)
    tol = (np.exp2(np.floor(np.log2(np.maximum(np.abs(fc), 1e-30))) - 7)).sum(axis=0) + \
        k * 2.0**-24 * 1.01 * (np.abs(fa).sum(axis=0) @ np.abs(fb))
    assert np.all(np.abs(fc.sum(axis=0) - colsum_exact) <= tol)
    for p in (da, db, dc):
        rt.free(p)


def test_gemm_m2_fp16_ragged_full(rt):
    # fp16 3000 x 4097 x 2050, elementwise against FP64
    m, n, k = 3000, 4097, 2050
    a = orc.uniform(m * k, 7, 1)
    b = orc.uniform(k * n, 8, 1)
    print("rel-L2", check(gpu_gemm(rt, a, b, m, n, k, 1), a, b, m, n, k, 1))
