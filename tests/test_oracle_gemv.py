"""CPU oracle GEMV: canonical order, reference order (gemv.cpp:126-134) and
FP64, pinned by closed forms, the reference's known-answer checks and error
bounds."""
import numpy as np
import pytest

import oracle_lib as orc


def f32(codes, dtype=0):
    return orc.decode(codes, dtype)


def test_canonical_order_pinned_by_absorption_pattern():
    # products 2^24 at one slot and 1 elsewhere: only the canonical
    # association (512 lane/slot accumulators, 8->1 fold, 64-lane butterfly)
    # yields 2^24 + 510: lane 0 folds ((2^24+1)+(1+1))+((1+1)+(1+1)) =
    # 2^24 + 6 (the first +1 is absorbed), the other 63 lanes give 8 each.
    k = 512
    a = np.ones(k, np.float32)
    x = np.ones(k, np.float32)
    a[0] = x[0] = 4096.0
    got = orc.lib().orc_canonical_dot(orc.ptr(orc.encode(a, 0)), orc.ptr(orc.encode(x, 0)), k, 0)
    assert got == 2.0**24 + 510
    # a sequential sum would absorb every +1
    seq = np.cumsum((a * x).astype(np.float32), dtype=np.float32)[-1]
    assert seq == 2.0**24


def test_canonical_order_slot_and_chunk_mapping():
    # big term at lane 5, slot 3 of chunk 1 (k = 512 + 5*8 + 3): that
    # accumulator holds 1 from chunk 0, and 1 + 2^24 rounds to 2^24.
    k = 1024
    a = np.ones(k, np.float32)
    x = np.ones(k, np.float32)
    big = 512 + 5 * 8 + 3
    a[big] = x[big] = 4096.0
    got = orc.lib().orc_canonical_dot(orc.ptr(orc.encode(a, 0)), orc.ptr(orc.encode(x, 0)), k, 0)
    # lane 5: slot 3 = 1 + 2^24 -> 2^24 ; other 7 slots = 2 each -> 14 ; = 2^24 + 14
    # lanes != 5: 16 each -> 63 * 16 = 1008 ; total 2^24 + 1022
    assert got == 2.0**24 + 1022


def test_canonical_sum_matches_exact_integer_sums():
    rng = np.random.default_rng(0)
    for n in (1, 7, 8, 511, 512, 513, 4096, 5000):
        t = rng.integers(-1000, 1000, n).astype(np.float32)
        assert orc.lib().orc_canonical_sum(orc.ptr(t), n) == float(t.astype(np.int64).sum())


def test_reference_order_is_sequential_fp32():
    rng = np.random.default_rng(1)
    m, k = 8, 3000
    a = orc.uniform(m * k, 5, 0)
    x = orc.uniform(k, 6, 0)
    got = orc.gemv_rows_seq(a, x, m, k, k, 0)
    fa = f32(a).reshape(m, k)
    fx = f32(x)
    for r in range(m):
        prod = (fa[r] * fx).astype(np.float32)
        assert got[r] == np.cumsum(prod, dtype=np.float32)[-1]


@pytest.mark.parametrize("dtype", [0, 1])
@pytest.mark.parametrize("m,k,lda", [(64, 4096, 4096), (37, 1000, 1000), (5, 1032, 1040), (300, 8, 8), (3, 1, 1)])
def test_canonical_within_fp32_error_bound_of_fp64(dtype, m, k, lda):
    a = orc.uniform(m * lda, 11 + k, dtype)
    x = orc.uniform(k, 12 + k, dtype)
    y = f32(orc.gemv_canonical(a, x, m, k, lda, dtype), dtype).astype(np.float64)
    exact = orc.gemv_f64(a, x, m, k, lda, dtype)
    absdot = np.abs(f32(a, dtype).reshape(m, lda)[:, :k].astype(np.float64)) @ np.abs(f32(x, dtype).astype(np.float64))
    u = 2.0**-24
    gamma = k * u / (1 - k * u)
    out_ulp = 2.0**-8 if dtype == 0 else 2.0**-11
    bound = gamma * absdot + np.abs(exact) * out_ulp + 1e-30
    assert np.all(np.abs(y - exact) <= bound * 1.0001)


def test_reference_known_answer_check_gemv_cpp():
    # gemv.cpp:91-103 inputs, first 64 rows, tolerance max(1, 1%) (:196-198)
    for dtype in (0, 1):
        m = k = 4096
        a, x = orc.reference_gemv_inputs(64, k, k, dtype)
        expected = orc.gemv_rows_seq(a, x, 64, k, k, dtype)
        got = f32(orc.gemv_canonical(a, x, 64, k, k, dtype), dtype)
        tol = np.maximum(1.0, np.abs(expected) * 0.01)
        assert np.all(np.abs(got - expected) <= tol)


def test_production_shapes_lane_order_equivalence():
    # qwen3/tests/test_cpu_reference.cpp:58-83 with the canonical order in
    # place of the 32-lane order, plus the Qwen3-0.6B shapes
    shapes = [(4096, 4096), (1024, 4096), (12288, 4096), (4096, 12288), (151936, 4096),
              (2048, 1024), (1024, 2048), (3072, 1024), (1024, 3072), (151936, 1024)]
    for rows, cols in shapes:
        kk = np.arange(cols)
        v = orc.encode(((kk % 17) - 8) / 128.0, 0)
        for row in (0, rows - 1):
            w = orc.encode((((row + kk) % 13) - 6) / 256.0, 0)
            expected = np.cumsum(f32(w) * f32(v), dtype=np.float32)[-1]
            got = f32(orc.gemv_canonical(w, v, 1, cols, cols, 0))[0]
            assert abs(got - expected) <= 0.03 + 0.02 * abs(expected)


def test_unit_vector_rows_select_entries():
    # A = identity rows -> y = x exactly (every other product is zero)
    k = 700
    x = orc.uniform(k, 9, 0)
    a = np.zeros((k, k), np.uint16)
    one = orc.encode(np.array([1.0], np.float32), 0)[0]
    a[np.arange(k), np.arange(k)] = one
    y = orc.gemv_canonical(a.ravel(), x, k, k, k, 0)
    fx = f32(x)
    assert np.array_equal(f32(y)[fx != 0], fx[fx != 0])
