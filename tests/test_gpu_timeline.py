"""The timestamps code object (build/xpu_kernels_stamps.hsaco, the product
kernels built with -DXPU_STAMPS) and its reader, xpu_playground_amd/timeline.py,
on the GPU: every launch is found, and the phase marks of the GEMM and the
decode attention split each wave's cycles into segments that add up to the
wave (the measurements behind profiles/gemm_and_attention_phase_cycles.md)."""
import argparse

import pytest

from xpu_playground_amd import timeline as tl

pytestmark = pytest.mark.gpu


def args(**kw):
    return argparse.Namespace(module=tl.STAMPS_MODULE, **kw)


def test_gemm_launches_and_phases():
    res = tl.run_gemm(args(size=4096, m=0, n=0, k=0, type="bf16", steps=3))
    assert len(res["launches"]) == 3  # one block per compute unit: no late blocks
    for ln in res["launches"]:
        ph = ln["phases"]
        assert ph is not None and ph["waves"] == 1024  # 256 blocks of 4 wavefronts
        segs = ph["median_cycles"]
        assert list(segs) == tl.PHASES["gemm"]
        assert all(v > 0 for v in segs.values()), segs
        # the K loop dominates, and the segments' medians add up to about
        # the median wave (each wave's segments add up to it exactly)
        assert segs[tl.PHASES["gemm"][1]] > 0.8 * ln["median_wave_cycles"]
        assert abs(sum(segs.values()) - ln["median_wave_cycles"]) <= 0.02 * ln["median_wave_cycles"]


def test_decode_launches_and_attention_phases():
    res = tl.run_decode(args(preset="qwen3-0.6b", prompt=16, new=4, mode="graph"))
    # 3 decode steps of 28 x 5 + 2 launches (the grouping by timestamps can
    # split a launch whose last blocks start late: at most a few extra)
    assert 28 * 5 + 2 <= res["kernels_per_token"] <= 28 * 5 + 3
    att = res["per_kernel"]["attention"]
    assert 28 * 3 <= att["launches"] <= 28 * 3 + 2
    segs = att["phases"]["median_cycles"]
    assert list(segs) == tl.PHASES["attention"]
    assert all(v > 0 for v in segs.values()), segs
    # only the 16 query-head blocks pass the marks
    assert att["phases"]["waves"] == 28 * 3 * 16 * 4
