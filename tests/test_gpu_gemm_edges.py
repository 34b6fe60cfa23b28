"""The GEMM's edge predication on gfx950: A and B are read in place for any
M, N, K and any 2-byte alignment (kernels/gemm.hip): the LDS-DMA stages
unaligned rows, the last K-slice's chunk that straddles column K is cut to
its live elements in LDS, and the two elements the buffer range check cuts
at the operands' ends (A[M-1][K-1] for odd K, B[K-1][N-1] for odd N) are put
back. The reference pads its operands with zeros on the host instead
(gemm.cpp:75-85); the results must be those of the zero-padded product.

Checked against the FP64 oracle at the GEMM bar (rel-L2 <= 1e-3, <= 2
output ulps + gamma_K sum|a b| per element), for every residue of K and N
mod 8 and each block tile, plus targeted values: an element past K that is
infinite (the next row's first element) must not reach the row before it,
and the restored elements are made large so that losing them fails."""
import numpy as np
import pytest

import oracle_lib as orc
import xpu_playground_amd as xpu
from test_gpu_gemm import check, gpu_gemm
from xpu_playground_amd import Args

pytestmark = pytest.mark.gpu

GUARD = 0x7E7E
TILES = {"": (256, 256), "_odd": (256, 256), "_m224": (224, 256), "_m224_odd": (224, 256), "_m128": (128, 256),
         "_t128": (128, 128)}


@pytest.mark.parametrize("dtype", [xpu.BF16, xpu.FP16])
@pytest.mark.parametrize("m,n,k", [(40, 33, k) for k in range(1, 18)] +
                         [(257, 129, 63), (130, 7, 65), (64, 1, 127), (1, 300, 130), (300, 257, 1001),
                          (3, 5, 2049)])
def test_ragged_shapes_through_xpu_gemm(rt, dtype, m, n, k):
    print(f"gemm edges dtype={dtype} {m}x{n}x{k}", flush=True)
    a = orc.uniform(m * k, 60 + m + k, dtype)
    b = orc.uniform(k * n, 70 + n + k, dtype)
    check(gpu_gemm(rt, a, b, m, n, k, dtype), a, b, m, n, k, dtype)


def launch_tile(rt, tag, dtype, a, b, m, n, k, offsets):
    """One launch of a tile variant by name on operands that start offsets
    = (a, b, c) bytes past a 16-byte boundary; guard codes around C."""
    bm, bn = TILES[tag]
    oa, ob, oc = offsets
    words = m * n + 32
    da, db, dc = rt.alloc(a.size * 2 + 32), rt.alloc(b.size * 2 + 32), rt.alloc(words * 2)
    try:
        rt.copy_to(da + oa, a)
        rt.copy_to(db + ob, b)
        rt.copy_to(dc, np.full(words, GUARD, np.uint16))
        c16 = oc % 16 == 0 and n % 8 == 0
        edge = "_edge" if k % 8 or n % 2 else ""
        name = f"xpu_gemm_{'fp16' if dtype else 'bf16'}{tag}_{'dma' if c16 else 'dmau'}{edge}"
        args = Args().ptr(da + oa).ptr(db + ob).ptr(dc + oc).u32(m).u32(n).u32(k).u32(k).u32(n).u32(n)
        grid = ((m + bm - 1) // bm) * ((n + bn - 1) // bn)
        print(f"{name} {m}x{n}x{k} offsets {offsets} grid {grid}", flush=True)
        rt.launch_grid(name, grid, 256, 0, args)
        rt.synchronize()
        out = rt.download(dc, words, np.uint16)
    finally:
        for p in (da, db, dc):
            rt.free(p)
    o = oc // 2
    assert np.all(out[:o] == GUARD) and np.all(out[o + m * n:] == GUARD), "store outside C"
    return out[o:o + m * n].reshape(m, n)


@pytest.mark.parametrize("tag", list(TILES))
@pytest.mark.parametrize("dtype", [xpu.BF16, xpu.FP16])
@pytest.mark.parametrize("m,n,k,offsets", [(300, 263, 201, (0, 0, 0)), (129, 77, 2050, (2, 6, 2)),
                                           (513, 9, 131, (10, 2, 0)), (255, 513, 67, (6, 14, 4)),
                                           (64, 40, 9, (2, 2, 2)), (257, 255, 1087, (0, 2, 6))])
def test_each_tile_in_place(rt, tag, dtype, m, n, k, offsets):
    slices = (k + 63) // 64
    if tag.endswith("_odd") and (slices % 2 == 0 or slices < 3):
        pytest.skip("the odd form takes an odd slice count of 3 or more")
    a = orc.uniform(m * k, 80 + m, dtype)
    b = orc.uniform(k * n, 90 + n, dtype)
    check(launch_tile(rt, tag, dtype, a, b, m, n, k, offsets), a, b, m, n, k, dtype)


@pytest.mark.parametrize("dtype", [xpu.BF16, xpu.FP16])
@pytest.mark.parametrize("m,n,k", [(9, 13, 11), (300, 7, 65), (257, 259, 2049)])
def test_values_past_k_do_not_leak_and_cut_elements_are_restored(rt, dtype, m, n, k):
    # Every odd row starts with +Inf: for the row before it that element sits
    # right after its last element, in the chunk that straddles K. Rows whose
    # own elements are finite must come out finite and within the bar.
    # K and N odd: A[M-1][K-1] and B[K-1][N-1] share a dword with the byte
    # past their operand; they are set to 64, so a lost element moves C by
    # 64 * |b| or 64 * |a|, far outside the bar.
    rng = np.random.default_rng(m + n + k)
    fa = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    fb = rng.uniform(-1, 1, (k, n)).astype(np.float32)
    fa[1::2, 0] = np.inf
    fa[m - 1, k - 1] = 64.0
    fb[k - 1, n - 1] = 64.0
    a = orc.encode(fa.reshape(-1), dtype)
    b = orc.encode(fb.reshape(-1), dtype)
    c = gpu_gemm(rt, a, b, m, n, k, dtype)
    finite_rows = np.array([r for r in range(m) if r % 2 == 0], np.int64)
    got = orc.decode(c[finite_rows], dtype)
    assert np.all(np.isfinite(got)), "an element past K reached the row before it"
    check(c, a, b, m, n, k, dtype, rows=finite_rows)
    # the rows that hold +Inf: every column gets +/-Inf or NaN, as the
    # zero-padded product would give
    assert not np.any(np.isfinite(orc.decode(c[1::2], dtype)))


def tile_shapes(count, seed):
    """Seeded shapes for which the 224 x 256 tile is a candidate: M and N
    of a few thousand, any K, ragged and aligned, with operand offsets."""
    rng = np.random.default_rng(seed)
    return [(int(rng.integers(1, 3600)), int(rng.integers(1, 4300)), int(rng.integers(1, 700)),
             tuple(int(x) for x in rng.choice([0, 2, 4, 6, 8, 10, 12, 14], 3))) for _ in range(count)]


@pytest.mark.parametrize("m,n,k,offsets", tile_shapes(12, 224))
def test_224_tile_equals_256_tile(rt, m, n, k, offsets):
    # the two wavefront arrangements run the same k-order in every MFMA
    # chain, so their outputs are the same bits (and stay inside C)
    dtype = xpu.FP16 if (m + n + k) % 2 else xpu.BF16
    odd = "_odd" if (k + 63) // 64 % 2 == 1 and (k + 63) // 64 >= 3 else ""
    a = orc.uniform(m * k, 3 * m + 1, dtype)
    b = orc.uniform(k * n, 5 * n + 2, dtype)
    big = launch_tile(rt, odd, dtype, a, b, m, n, k, offsets)
    assert np.array_equal(launch_tile(rt, "_m224" + odd, dtype, a, b, m, n, k, offsets), big)


def test_ragged_baseline_shape_reads_operands_in_place(rt):
    # configs[3] (fp16 3000 x 4097 x 2050) with A and B at 2-byte offsets,
    # all 12.3 M outputs against FP64
    m, n, k = 3000, 4097, 2050
    a = orc.uniform(m * k, 7, xpu.FP16)
    b = orc.uniform(k * n, 8, xpu.FP16)
    out = launch_tile(rt, "_odd", xpu.FP16, a, b, m, n, k, (2, 2, 2))
    print("rel-L2", check(out, a, b, m, n, k, xpu.FP16), flush=True)
    # the 224 x 256 tile (the one xpu_gemm picks here): the same bits
    assert np.array_equal(launch_tile(rt, "_m224_odd", xpu.FP16, a, b, m, n, k, (2, 2, 2)), out)


@pytest.mark.parametrize("dtype", [xpu.BF16, xpu.FP16])
@pytest.mark.parametrize("m,n,k,c_offset", [(1024, 1024, 4096, 0), (512, 512, 2048, 0), (300, 201, 1030, 2),
                                            (129, 383, 2049, 6), (64, 8, 512, 0), (512, 512, 512, 2)])
def test_split_k_products(rt, dtype, m, n, k, c_offset):
    # Outputs that leave most compute units idle with 128 x 128 tiles and a
    # long enough reduction are split over the idle units (FP32 partials
    # added in split order): within the GEMM bar against FP64, written
    # exactly over C (guard codes around it), on 16-byte and unaligned C
    print(f"gemm split-K dtype={dtype} {m}x{n}x{k} C offset {c_offset}", flush=True)
    a = orc.uniform(m * k, 100 + m, dtype)
    b = orc.uniform(k * n, 110 + n, dtype)
    da, db = rt.upload(a), rt.upload(b)
    words = m * n + 32
    dc = rt.alloc(words * 2)
    try:
        rt.copy_to(dc, np.full(words, GUARD, np.uint16))
        rt.gemm(dtype, da, db, dc + c_offset, m, n, k)
        rt.synchronize()
        out = rt.download(dc, words, np.uint16)
    finally:
        for p in (da, db, dc):
            rt.free(p)
    o = c_offset // 2
    assert np.all(out[:o] == GUARD) and np.all(out[o + m * n:] == GUARD), "store outside C"
    rows = None if m * n <= 512 * 512 else np.arange(0, m, 7)
    check(out[o:o + m * n].reshape(m, n), a, b, m, n, k, dtype, rows=rows)
