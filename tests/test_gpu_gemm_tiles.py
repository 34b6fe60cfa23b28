"""The GEMM's block tiles (256x256 and 224x256, also in their
odd-slice-count forms; 128x256, the reference's small tile of
gemm_kernel.hpp:26-27; 128x128)
launched by name on the same shapes, each against the FP64 oracle at the GEMM
bar, with 16-byte and 2-byte-offset C; and the tile xpu_gemm picks
(gemm.cpp:145's choice, made here by compute-unit fill)."""
import numpy as np
import pytest

import oracle_lib as orc
import xpu_playground_amd as xpu
from test_gpu_gemm import check, gpu_gemm
from xpu_playground_amd import Args

pytestmark = pytest.mark.gpu

# "_odd": the 256x256 and 224x256 kernels for an odd number (3 or more) of
# 64-deep K-slices (the last slice on its own after the pairs, only its
# k-steps below K); launched only on such K, as xpu_gemm does
TILES = {"": (256, 256), "_odd": (256, 256), "_m224": (224, 256), "_m224_odd": (224, 256), "_m128": (128, 256),
         "_t128": (128, 128)}


def slices(k):
    return (k + 63) // 64
GUARD = 0x7E7E


def launch_tile(rt, tag, dtype, a, b, m, n, k, c_offset):
    """One launch of a tile variant on 16-byte aligned A and B (K and N
    multiples of 8 here; ragged shapes and offsets: test_gpu_gemm_edges.py);
    C starts c_offset bytes past a 16-byte boundary (the _dmau stores for 2)."""
    assert k % 8 == 0 and n % 8 == 0 and a.size == m * k and b.size == k * n
    bm, bn = TILES[tag]
    words = m * n + 32
    da, db, dc = rt.upload(a), rt.upload(b), rt.alloc(words * 2)
    try:
        rt.copy_to(dc, np.full(words, GUARD, np.uint16))
        name = f"xpu_gemm_{'fp16' if dtype else 'bf16'}{tag}_{'dmau' if c_offset else 'dma'}"
        args = Args().ptr(da).ptr(db).ptr(dc + c_offset).u32(m).u32(n).u32(k).u32(k).u32(n).u32(n)
        grid = ((m + bm - 1) // bm) * ((n + bn - 1) // bn)
        print(f"{name} {m}x{n}x{k} grid {grid}", flush=True)
        rt.launch_grid(name, grid, 256, 0, args)
        rt.synchronize()
        out = rt.download(dc, words, np.uint16)
    finally:
        for p in (da, db, dc):
            rt.free(p)
    off = c_offset // 2
    assert np.all(out[:off] == GUARD) and np.all(out[off + m * n:] == GUARD), "store outside C"
    return out[off:off + m * n].reshape(m, n)


@pytest.mark.parametrize("tag", list(TILES))
@pytest.mark.parametrize("dtype", [xpu.BF16, xpu.FP16])
@pytest.mark.parametrize("c_offset", [0, 2])
@pytest.mark.parametrize("m,n,k", [(128, 128, 64), (255, 264, 72), (37, 56, 8), (300, 8, 16), (513, 392, 1032),
                                   (1000, 600, 520), (255, 264, 136), (300, 8, 184), (64, 520, 1056)])
def test_tile_variant(rt, tag, dtype, c_offset, m, n, k):
    if tag.endswith("_odd") and (slices(k) % 2 == 0 or slices(k) < 3):
        pytest.skip("the odd form takes an odd slice count of 3 or more")
    a = orc.uniform(m * k, 50 + m, dtype)
    b = orc.uniform(k * n, 60 + n, dtype)
    check(launch_tile(rt, tag, dtype, a, b, m, n, k, c_offset), a, b, m, n, k, dtype)


def test_tiles_same_bits(rt):
    # every tile runs the same k-order in each MFMA chain, so all of them
    # give the same output bits
    m, n, k = 700, 520, 1064  # 17 slices, 3 live k-steps in the last
    a = orc.uniform(m * k, 71, xpu.BF16)
    b = orc.uniform(k * n, 72, xpu.BF16)
    outs = [launch_tile(rt, tag, xpu.BF16, a, b, m, n, k, 0) for tag in TILES]
    assert all(np.array_equal(outs[0], o) for o in outs[1:])


def test_tile_choice(rt):
    if rt.compute_units != 256:
        pytest.skip("the expected choices are for MI355X's 256 compute units")
    # configs[2] keeps the large tile (it gives every compute unit one
    # block); configs[3] takes 224 x 256 (238 blocks of 7/8 the work instead
    # of 204); outputs that leave most units idle take a small one
    assert rt.gemm_tile(4096, 4096) == (256, 256)
    assert rt.gemm_tile(3000, 4097) == (224, 256)
    assert rt.gemm_tile(3072, 3072) == (224, 256)
    assert rt.gemm_tile(6144, 6144) == (224, 256)  # three blocks per unit with either large tile
    assert rt.gemm_tile(8192, 8192) == (256, 256)
    assert rt.gemm_tile(2048, 4096) == (128, 256)
    assert rt.gemm_tile(1000, 4097) == (128, 256)
    assert rt.gemm_tile(2048, 2048) == (128, 128)
    assert rt.gemm_tile(1024, 1024) == (128, 128)
    assert rt.gemm_tile(1, 1) == (128, 128)


@pytest.mark.parametrize("m,n,k", [(1024, 1024, 1024), (2048, 4096, 256), (1000, 4097, 520), (777, 1001, 300)])
def test_small_tile_shapes_through_xpu_gemm(rt, m, n, k):
    # operands read in place, aligned and ragged (unaligned C rows with N % 8 != 0)
    print(f"xpu_gemm {m}x{n}x{k} tile {rt.gemm_tile(m, n)}", flush=True)
    a = orc.uniform(m * k, 80 + m, xpu.BF16)
    b = orc.uniform(k * n, 90 + n, xpu.BF16)
    check(gpu_gemm(rt, a, b, m, n, k, xpu.BF16), a, b, m, n, k, xpu.BF16)


def random_shapes(count, seed):
    """Seeded shapes across every launch form: small outputs (128x128 and
    128x256 tiles), outputs that fill the chip with 256x256 tiles (short K,
    so the FP64 oracle stays within a few seconds), ragged M, N and K
    (padding, unaligned C), and odd and even slice counts."""
    rng = np.random.default_rng(seed)
    regimes = [((1, 1200), (1, 1200), (1, 1400)), ((1400, 2700), (1400, 4200), (8, 700)),
               ((2800, 4200), (2800, 4200), (8, 400))]
    shapes = []
    for i in range(count):
        (m0, m1), (n0, n1), (k0, k1) = regimes[i % 3]
        shapes.append((int(rng.integers(m0, m1)), int(rng.integers(n0, n1)), int(rng.integers(k0, k1))))
    return shapes


@pytest.mark.parametrize("m,n,k", random_shapes(24, 2026))
def test_gemm_random_shapes(rt, m, n, k):
    print(f"xpu_gemm {m}x{n}x{k} tile {rt.gemm_tile(m, n)}", flush=True)
    dtype = xpu.FP16 if (m + n + k) % 2 else xpu.BF16
    a = orc.uniform(m * k, 7 * m + 1, dtype)
    b = orc.uniform(k * n, 11 * n + 2, dtype)
    check(gpu_gemm(rt, a, b, m, n, k, dtype), a, b, m, n, k, dtype)
