"""GEMV on gfx950 vs the CPU oracle: bit-exact against the canonical order,
and within BASELINE's bar (rel-L2 <= 1e-3, <= 2 output ulps beyond the FP32
rounding bound) against FP64."""
import numpy as np
import pytest

import oracle_lib as orc
import xpu_playground_amd as xpu

pytestmark = pytest.mark.gpu


def gpu_gemv(rt, a, x, m, k, lda, dtype):
    da, dx = rt.upload(a), rt.upload(x)
    dy = rt.alloc(m * 2)
    try:
        rt.gemv(dtype, da, dx, dy, m, k, lda)
        rt.synchronize()
        return rt.download(dy, m, np.uint16)
    finally:
        for p in (da, dx, dy):
            rt.free(p)


def check_against_fp64(y, a, x, m, k, lda, dtype):
    """BASELINE's bar: against the accumulated reference rounded to the output
    type (here the FP64 sum, the FP32-accumulated value's exact limit),
    rel-L2 <= 1e-3 and |error| <= 2 output ulps plus the FP32 accumulation
    bound gamma_K * sum|a x| (which matters only for outputs near zero)."""
    exact = orc.gemv_f64(a, x, m, k, lda, dtype)
    ref = orc.decode(orc.encode(exact.astype(np.float32), dtype), dtype).astype(np.float64)
    got = orc.decode(y, dtype).astype(np.float64)
    rel_l2 = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-300)
    assert rel_l2 <= 1e-3, rel_l2
    absdot = np.abs(orc.decode(a, dtype).reshape(m, lda)[:, :k].astype(np.float64)) @ np.abs(
        orc.decode(x, dtype).astype(np.float64))
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(ref), 1e-30))) - (7 if dtype == 0 else 10))
    gamma = k * 2.0**-24 / (1 - k * 2.0**-24)
    assert np.all(np.abs(got - ref) <= 2 * ulp + gamma * absdot)
    return rel_l2


SHAPES = [
    (1, 1, 1), (3, 5, 5), (64, 512, 512), (37, 1000, 1000), (1000, 1032, 1040), (33, 4097, 4097),
    (4096, 1024, 1024), (1024, 3072, 3072), (151936, 1024, 1024), (8191, 2050, 2050),
    # two rows per wavefront (K <= 8192, aligned) with an odd row count: the
    # last wavefront's second row is past M
    (4095, 2048, 2048), (7, 8192, 8200), (1025, 8200, 8200),
]


@pytest.mark.parametrize("dtype", [xpu.BF16, xpu.FP16])
@pytest.mark.parametrize("m,k,lda", SHAPES)
def test_gemv_matches_oracle(rt, dtype, m, k, lda):
    print(f"gemv dtype={dtype} m={m} k={k} lda={lda}", flush=True)
    a = orc.uniform(m * lda, 100 + m, dtype)
    x = orc.uniform(k, 200 + k, dtype)
    y = gpu_gemv(rt, a, x, m, k, lda, dtype)
    assert np.array_equal(y, orc.gemv_canonical(a, x, m, k, lda, dtype))
    check_against_fp64(y, a, x, m, k, lda, dtype)


@pytest.mark.parametrize("dtype", [xpu.BF16, xpu.FP16])
@pytest.mark.parametrize("m,k,lda", [(64, 512, 512), (37, 1000, 1000), (1000, 1032, 1040), (5, 3, 7)])
def test_gemv_pointers_two_bytes_past_alignment(rt, dtype, m, k, lda):
    # A, x and y start 2 bytes past a 16-byte boundary, which the 16-byte
    # loads of the vector variants cannot take: the 16-bit-load variant runs.
    # Guard codes around y catch any store outside it.
    print(f"gemv unaligned pointers dtype={dtype} m={m} k={k} lda={lda}", flush=True)
    a = orc.uniform(m * lda, 300 + m, dtype)
    x = orc.uniform(k, 400 + k, dtype)
    guard = 0x7E7E
    pa, px, py = rt.alloc(m * lda * 2 + 64), rt.alloc(k * 2 + 64), rt.alloc(m * 2 + 64)
    try:
        rt.copy_to(py, np.full((m * 2 + 64) // 2, guard, np.uint16))
        rt.copy_to(pa + 2, a)
        rt.copy_to(px + 2, x)
        rt.gemv(dtype, pa + 2, px + 2, py + 2, m, k, lda)
        rt.synchronize()
        out = rt.download(py, (m * 2 + 64) // 2, np.uint16)
    finally:
        for p in (pa, px, py):
            rt.free(p)
    assert out[0] == guard and np.all(out[1 + m:] == guard)
    assert np.array_equal(out[1:1 + m], orc.gemv_canonical(a, x, m, k, lda, dtype))


def test_gemv_large_k_reads_vector_from_global(rt):
    m, k = 8, 100000
    a = orc.uniform(m * k, 7, 0)
    x = orc.uniform(k, 8, 0)
    y = gpu_gemv(rt, a, x, m, k, k, 0)
    assert np.array_equal(y, orc.gemv_canonical(a, x, m, k, k, 0))


def test_device_fill_matches_oracle_generator(rt):
    for dtype in (0, 1):
        n = 1_000_003
        p = rt.alloc(n * 2)
        rt.fill_uniform(dtype, p, n, 77)
        rt.synchronize()
        assert np.array_equal(rt.download(p, n, np.uint16), orc.uniform(n, 77, dtype))
        rt.free(p)


def test_gemv_v1_bf16_4096_full_parity(rt):
    # bf16 4096 x 4096, seeded U[-1,1], device-generated
    m = k = 4096
    da, dx, dy = rt.alloc(m * k * 2), rt.alloc(k * 2), rt.alloc(m * 2)
    rt.fill_uniform(0, da, m * k, 1)
    rt.fill_uniform(0, dx, k, 2)
    rt.gemv(0, da, dx, dy, m, k, k)
    rt.synchronize()
    a = rt.download(da, m * k, np.uint16)
    x = rt.download(dx, k, np.uint16)
    y = rt.download(dy, m, np.uint16)
    assert np.array_equal(a[:1 << 20], orc.uniform(1 << 20, 1, 0))
    assert np.array_equal(y, orc.gemv_canonical(a, x, m, k, k, 0))
    print("rel-L2", check_against_fp64(y, a, x, m, k, k, 0))
    for p in (da, dx, dy):
        rt.free(p)


def test_gemv_v2_fp16_16384_full_parity(rt):
    # fp16 16384 x 16384 (512 MiB matrix)
    m = k = 16384
    da, dx, dy = rt.alloc(m * k * 2), rt.alloc(k * 2), rt.alloc(m * 2)
    rt.fill_uniform(1, da, m * k, 3)
    rt.fill_uniform(1, dx, k, 4)
    rt.gemv(1, da, dx, dy, m, k, k)
    rt.synchronize()
    a = rt.download(da, m * k, np.uint16)
    x = rt.download(dx, k, np.uint16)
    y = rt.download(dy, m, np.uint16)
    assert np.array_equal(x, orc.uniform(k, 4, 1))
    assert np.array_equal(y, orc.gemv_canonical(a, x, m, k, k, 1))
    rows = 2048  # FP64 statistics on a row sample keep the test short
    print("rel-L2", check_against_fp64(y[:rows], a[:rows * k], x, rows, k, k, 1))
    for p in (da, dx, dy):
        rt.free(p)


def test_reference_hash_init_known_answer(rt):
    # gemv.cpp:91-103 inputs on the device, check of :119-134
    for dtype in (0, 1):
        m, k = 256, 4096
        da, dx, dy = rt.alloc(m * k * 2), rt.alloc(k * 2), rt.alloc(m * 2)
        rt.fill_reference_gemv(dtype, da, dx, m, k, k)
        rt.gemv(dtype, da, dx, dy, m, k, k)
        rt.synchronize()
        a_ref, x_ref = orc.reference_gemv_inputs(m, k, k, dtype)
        assert np.array_equal(rt.download(da, m * k, np.uint16), a_ref)
        assert np.array_equal(rt.download(dx, k, np.uint16), x_ref)
        y = orc.decode(rt.download(dy, m, np.uint16), dtype)
        expected = orc.gemv_rows_seq(a_ref, x_ref, 64, k, k, dtype)
        assert np.all(np.abs(y[:64] - expected) <= np.maximum(1.0, 0.01 * np.abs(expected)))
        for p in (da, dx, dy):
            rt.free(p)


def test_gemv_every_input_code_round_trips(rt):
    # K = 1, x = 1: y = fl(+0 + a * 1) for all 65536 codes of A
    for dtype in (0, 1):
        codes = np.arange(65536, dtype=np.uint16)
        one = orc.encode(np.array([1.0], np.float32), dtype)
        y = gpu_gemv(rt, codes, one, 65536, 1, 1, dtype)
        vals = orc.decode(codes, dtype)
        keep = ~np.isnan(vals)
        assert np.array_equal(y[keep], orc.gemv_canonical(codes, one, 65536, 1, 1, dtype)[keep])
        ident = keep & (codes != 0x8000)
        assert np.array_equal(y[ident], codes[ident])
