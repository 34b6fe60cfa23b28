"""The GEMM's [n][k]-weight forms (C = A W^T, W row-major N x K as a
projection's weight is stored) and their residual forms (C = bf16(C +
bf16(A W^T))), launched by name for every tile against the FP64 oracle:
the GEMM bar for C = A W^T, and for the residual form the same bar on the
product plus one output ulp for the final addition."""
import numpy as np
import pytest

import oracle_lib as orc
import xpu_playground_amd as xpu
from test_gpu_gemm import check
from test_gpu_gemm_tiles import GUARD, TILES, launch_tile, slices
from xpu_playground_amd import Args

pytestmark = pytest.mark.gpu

# the [n][k] kernels: the [k][n] tiles except 224 x 256, plus 128 x 64,
# which only the [n][k] form has
NT_TILES = {**{t: v for t, v in TILES.items() if not t.startswith("_m224")}, "_n64": (128, 64)}


def launch_nt(rt, tag, res, a, w, c0, m, n, k):
    assert k % 8 == 0 and n % 8 == 0 and a.size == m * k and w.size == n * k and c0.size == m * n
    bm, bn = NT_TILES[tag]
    words = m * n + 16
    da, dw, dc = rt.upload(a), rt.upload(w), rt.alloc(words * 2)
    try:
        rt.copy_to(dc, np.concatenate([c0, np.full(16, GUARD, np.uint16)]))
        name = f"xpu_gemm_bf16{tag}_nt{'_res' if res else ''}_dma"
        args = Args().ptr(da).ptr(dw).ptr(dc).u32(m).u32(n).u32(k).u32(k).u32(n).u32(n)
        grid = ((m + bm - 1) // bm) * ((n + bn - 1) // bn)
        print(f"{name} {m}x{n}x{k} grid {grid}", flush=True)
        rt.launch_grid(name, grid, 256, 0, args)
        rt.synchronize()
        out = rt.download(dc, words, np.uint16)
    finally:
        for p in (da, dw, dc):
            rt.free(p)
    assert np.all(out[m * n:] == GUARD), "store past C"
    return out[:m * n].reshape(m, n)


def check_residual(got, old, a, w, m, n, k):
    """got = bf16(old + bf16(A W^T)): against old + the exact product, within
    the GEMM bar on the product (2 ulps of it + gamma_K sum|a w|) and one
    ulp of the output for the addition's rounding and the product's own."""
    wt = np.ascontiguousarray(w.reshape(n, k).T).reshape(-1)
    exact = orc.gemm_f64(a, wt, m, n, k, xpu.BF16)
    old_f = orc.decode(old, xpu.BF16).reshape(m, n).astype(np.float64)
    want = old_f + exact
    g = orc.decode(got, xpu.BF16).astype(np.float64)
    # rel-L2 against the same two roundings applied to the exact product
    prod = orc.decode(orc.encode(exact.astype(np.float32), xpu.BF16), xpu.BF16).astype(np.float64)
    ref = orc.decode(orc.encode((old_f + prod).astype(np.float32), xpu.BF16), xpu.BF16).astype(np.float64)
    rel = np.linalg.norm(g - ref) / max(np.linalg.norm(ref), 1e-300)
    assert rel <= 1e-3, rel

    def ulp(x):
        return np.exp2(np.floor(np.log2(np.maximum(np.abs(x), 1e-30))) - 7)
    absab = (np.abs(orc.decode(a, xpu.BF16).reshape(m, k).astype(np.float64))
             @ np.abs(orc.decode(wt, xpu.BF16).reshape(k, n).astype(np.float64)))
    gamma = k * 2.0**-24 / (1 - k * 2.0**-24)
    bound = ulp(want) + 2.5 * ulp(exact) + gamma * absab
    bad = np.abs(g - want) > bound
    assert not bad.any(), (int(bad.sum()), np.argwhere(bad)[:5])


SHAPES = [(128, 128, 64), (255, 264, 72), (37, 56, 8), (300, 8, 16), (513, 392, 1032), (255, 264, 136),
          (64, 520, 1056), (256, 4096, 1024), (256, 1024, 3072)]


@pytest.mark.parametrize("tag", list(NT_TILES))
@pytest.mark.parametrize("res", [False, True])
@pytest.mark.parametrize("m,n,k", SHAPES)
def test_nt_variant(rt, tag, res, m, n, k):
    if tag == "_odd" and (slices(k) % 2 == 0 or slices(k) < 3):
        pytest.skip("the odd form takes an odd slice count of 3 or more")
    a = orc.uniform(m * k, 150 + m, xpu.BF16)
    w = orc.uniform(n * k, 160 + n, xpu.BF16)
    old = orc.uniform(m * n, 170 + k, xpu.BF16) if res else np.full(m * n, GUARD, np.uint16)
    got = launch_nt(rt, tag, res, a, w, old, m, n, k)
    if res:
        check_residual(got, old, a, w, m, n, k)
    else:
        wt = np.ascontiguousarray(w.reshape(n, k).T).reshape(-1)
        check(got, a, wt, m, n, k, xpu.BF16)


def test_nt_same_bits_as_kn(rt):
    # the [n][k] form feeds the MFMAs the same products in the same order as
    # the [k][n] form on W^T, so the outputs are bitwise equal
    m, n, k = 700, 520, 1064
    a = orc.uniform(m * k, 171, xpu.BF16)
    w = orc.uniform(n * k, 172, xpu.BF16)
    wt = np.ascontiguousarray(w.reshape(n, k).T).reshape(-1)
    ref = launch_tile(rt, "", xpu.BF16, a, wt, m, n, k, 0)
    for tag in NT_TILES:
        if tag == "_odd" and slices(k) % 2 == 0:
            continue
        got = launch_nt(rt, tag, False, a, w, np.zeros(m * n, np.uint16), m, n, k)
        assert np.array_equal(got, ref), tag


def launch_splitk(rt, res, a, w, c0, m, n, k, spl):
    """The split-K form: xpu_gemm_bf16_n64_nt_part_dma over K ranges of spl
    slices (a multiple of 4), then xpu_gemm_splitk_reduce."""
    assert k % 8 == 0 and n % 8 == 0 and spl % 4 == 0
    slices = (k + 63) // 64
    splits = (slices + spl - 1) // spl
    tiles = ((m + 127) // 128) * ((n + 63) // 64)
    words = m * n + 16
    da, dw, dc = rt.upload(a), rt.upload(w), rt.alloc(words * 2)
    dp = rt.alloc(splits * m * n * 4)
    try:
        rt.copy_to(dc, np.concatenate([c0, np.full(16, GUARD, np.uint16)]))
        print(f"split-K {m}x{n}x{k} spl {spl} splits {splits} res {res}", flush=True)
        args = Args().ptr(da).ptr(dw).ptr(dp).u32(m).u32(n).u32(k).u32(spl).u32(n).u32(n)
        rt.launch_grid("xpu_gemm_bf16_n64_nt_part_dma", tiles * splits, 256, 0, args)
        rargs = Args().ptr(dp).ptr(dc).u32(m).u32(n).u32(splits).u32(1 if res else 0)
        rt.launch_grid("xpu_gemm_splitk_reduce", max(1, min((m * n // 8 + 255) // 256, 2048)), 256, 0, rargs)
        rt.synchronize()
        out = rt.download(dc, words, np.uint16)
    finally:
        for p in (da, dw, dc, dp):
            rt.free(p)
    assert np.all(out[m * n:] == GUARD), "store past C"
    return out[:m * n].reshape(m, n)


@pytest.mark.parametrize("res", [False, True])
@pytest.mark.parametrize("m,n,k,spl", [(127, 1024, 3072, 4), (511, 1024, 2048, 8), (127, 4096, 1024, 4), (37, 56, 200, 4),
                                       (300, 8, 1032, 8), (1, 64, 64, 4)])
def test_splitk(rt, res, m, n, k, spl):
    a = orc.uniform(m * k, 200 + m, xpu.BF16)
    w = orc.uniform(n * k, 210 + n, xpu.BF16)
    old = orc.uniform(m * n, 220 + k, xpu.BF16) if res else np.full(m * n, GUARD, np.uint16)
    got = launch_splitk(rt, res, a, w, old, m, n, k, spl)
    if res:
        check_residual(got, old, a, w, m, n, k)
    else:
        wt = np.ascontiguousarray(w.reshape(n, k).T).reshape(-1)
        check(got, a, wt, m, n, k, xpu.BF16)


@pytest.mark.parametrize("m,n,k,spl", [(127, 1024, 3072, 4), (300, 512, 1032, 4), (1, 1024, 256, 4),
                                       (129, 1024, 3072, 8), (64, 512, 4096, 4)])
def test_splitk_reduce_norm(rt, m, n, k, spl):
    # the reduction fused with the RMSNorm of its rows writes the same C as
    # xpu_gemm_splitk_reduce and the same normalised rows as
    # xpu_q3_pf_rmsnorm on that C, bit for bit
    slices = (k + 63) // 64
    splits = (slices + spl - 1) // spl
    tiles = ((m + 127) // 128) * ((n + 63) // 64)
    a = orc.uniform(m * k, 230 + m, xpu.BF16)
    w = orc.uniform(n * k, 240 + n, xpu.BF16)
    old = orc.uniform(m * n, 250 + k, xpu.BF16)
    gains = orc.encode(1.0 + 0.1 * orc.decode(orc.uniform(n, 260, xpu.BF16), xpu.BF16), xpu.BF16)
    eps = 1e-6
    da, dw, dg = rt.upload(a), rt.upload(w), rt.upload(gains)
    dc1, dc2 = rt.upload(old), rt.upload(old)
    dx1, dx2 = rt.alloc(m * n * 2), rt.alloc(m * n * 2)
    dp = rt.alloc(splits * m * n * 4)
    try:
        print(f"split-K reduce + norm {m}x{n}x{k} spl {spl} splits {splits}", flush=True)
        args = Args().ptr(da).ptr(dw).ptr(dp).u32(m).u32(n).u32(k).u32(spl).u32(n).u32(n)
        rt.launch_grid("xpu_gemm_bf16_n64_nt_part_dma", tiles * splits, 256, 0, args)
        rt.launch_grid("xpu_gemm_splitk_reduce_norm", (m + 3) // 4, 256, 0,
                       Args().ptr(dp).ptr(dc1).u32(m).u32(n).u32(splits).u32(1).ptr(dg).ptr(dx1).f32(eps))
        rt.launch_grid("xpu_gemm_splitk_reduce", max(1, min((m * n // 8 + 255) // 256, 2048)), 256, 0,
                       Args().ptr(dp).ptr(dc2).u32(m).u32(n).u32(splits).u32(1))
        rt.launch_grid("xpu_q3_pf_rmsnorm", (m + 3) // 4, 256, 0,
                       Args().ptr(dc2).ptr(dg).ptr(dx2).u32(n).f32(eps).u32(m))
        rt.synchronize()
        c1, c2 = rt.download(dc1, m * n, np.uint16), rt.download(dc2, m * n, np.uint16)
        x1, x2 = rt.download(dx1, m * n, np.uint16), rt.download(dx2, m * n, np.uint16)
    finally:
        for p in (da, dw, dg, dc1, dc2, dx1, dx2, dp):
            rt.free(p)
    assert np.array_equal(c1, c2)
    assert np.array_equal(x1, x2)
    check_residual(c1.reshape(m, n), old, a, w, m, n, k)
