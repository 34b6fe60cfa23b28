"""CPU oracle GEMM (FP64 and the reference's FP32 ascending-k order)."""
import numpy as np

import oracle_lib as orc


def test_constant_known_answer_gemm_cpp():
    # gemm.cpp:81-85,109-117: A = 0.5, B = 0.25 -> every C = 0.125 * K
    for m, n, k in [(64, 96, 4096), (3, 5, 2050)]:
        a = orc.encode(np.full(m * k, 0.5, np.float32), 0)
        b = orc.encode(np.full(k * n, 0.25, np.float32), 0)
        assert np.all(orc.gemm_f64(a, b, m, n, k, 0) == 0.125 * k)
        assert np.all(orc.gemm_f32_rows(a, b, m, n, k, 0, np.arange(m)) == 0.125 * k)


def test_f64_matches_numpy_float64_on_ragged_shapes():
    for dtype, (m, n, k) in [(0, (37, 53, 70)), (1, (30, 41, 129)), (0, (1, 1, 1))]:
        a = orc.uniform(m * k, 1, dtype)
        b = orc.uniform(k * n, 2, dtype)
        fa = orc.decode(a, dtype).reshape(m, k).astype(np.float64)
        fb = orc.decode(b, dtype).reshape(k, n).astype(np.float64)
        ref = fa @ fb
        got = orc.gemm_f64(a, b, m, n, k, dtype)
        assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)
        rows = np.array([m - 1, 0])
        assert np.allclose(orc.gemm_f64(a, b, m, n, k, dtype, rows), ref[rows], rtol=1e-12, atol=1e-12)


def test_identity_and_permutation_invariants():
    k = 64
    eye = orc.encode(np.eye(k, dtype=np.float32).ravel(), 0)
    b = orc.uniform(k * 33, 4, 0)
    assert np.array_equal(orc.gemm_f64(eye, b, k, 33, k, 0), orc.decode(b, 0).reshape(k, 33).astype(np.float64))
    perm = np.random.default_rng(0).permutation(k)
    p = np.zeros((k, k), np.float32)
    p[np.arange(k), perm] = 1
    got = orc.gemm_f64(orc.encode(p.ravel(), 0), b, k, 33, k, 0)
    assert np.array_equal(got, orc.decode(b, 0).reshape(k, 33)[perm].astype(np.float64))


def test_f32_rows_sequential_order():
    m, n, k = 4, 7, 500
    a = orc.uniform(m * k, 5, 0)
    b = orc.uniform(k * n, 6, 0)
    got = orc.gemm_f32_rows(a, b, m, n, k, 0, np.arange(m))
    fa = orc.decode(a, 0).reshape(m, k)
    fb = orc.decode(b, 0).reshape(k, n)
    for i in range(m):
        for j in range(n):
            assert got[i, j] == np.cumsum((fa[i] * fb[:, j]).astype(np.float32), dtype=np.float32)[-1]


def test_blocked_f32_equals_the_row_order_bitwise():
    # the GEMM CPU baseline (orc_gemm_f32_blocked) performs the row version's
    # sums: ascending k per element, FP32, across the 64 x 512 x 256 blocks
    for dtype, (m, n, k) in [(0, (70, 600, 300)), (1, (65, 513, 257)), (0, (1, 3, 1))]:
        a = orc.uniform(m * k, 7, dtype)
        b = orc.uniform(k * n, 8, dtype)
        rows = orc.gemm_f32_rows(a, b, m, n, k, dtype, np.arange(m))
        blocked = np.empty((m, n), np.float32)
        orc.lib().orc_gemm_f32_blocked(orc.ptr(a), orc.ptr(b), orc.ptr(blocked), m, n, k, dtype)
        assert np.array_equal(rows, blocked)
