"""The stamps reader (xpu_playground_amd/timeline.py) on synthetic records:
launch grouping by kernel id and overlap, and the phase segments derived
from the XPU_PHASE marks (entry to the first mark, mark to mark, last mark to
exit; waves that pass no mark left out)."""
import numpy as np

from xpu_playground_amd import timeline as tl


def records(rows):
    """rows: (start, real_ticks, clock_ticks, kernel, block, phases)."""
    out = np.zeros(len(rows), dtype=[("real_start", "<i8"), ("real_ticks", "<u4"), ("clock_ticks", "<u4"),
                                      ("kernel", "<u4"), ("xcc", "<u4"), ("block", "<u4"),
                                      ("phases", "<u4", (tl.PHASE_COUNT,))])
    for i, (s, rt, ct, k, b, ph) in enumerate(rows):
        out[i] = (s, rt, ct, k, b % 8, b, ph)
    return out


def test_launch_grouping_and_gaps():
    recs = records([
        (0, 100, 200, 2, 0, (10, 150, 160, 0)),
        (5, 100, 210, 2, 1, (12, 160, 170, 0)),
        (300, 50, 100, 2, 0, (0, 0, 0, 0)),   # enters after every wave of the first launch left
        (310, 20, 40, 11, 0, (0, 0, 0, 0)),   # another kernel id
    ])
    lns = tl.launches(recs)
    assert [ln["name"] for ln in lns] == ["gemm", "gemm", "attention"]
    assert lns[0]["waves"] == 2 and lns[0]["end"] == 105
    assert abs(lns[1]["gap_us"] - (300 - 105) * tl.TICK_NS / 1e3) < 1e-9
    assert len(lns[0]["marks"]) == 2 and lns[1]["marks"] == []


def test_phase_segments_are_differences_of_marks():
    # three marks and the exit: segments 10, 140, 10, 40 and 12, 148, 10, 40
    marks = [[10, 150, 160, 0, 200], [12, 160, 170, 0, 210]]
    assert tl.phase_segments(marks) == [11.0, 144.0, 10.0, 40.0]
    # a wave that missed a mark the others passed is left out
    assert tl.phase_segments(marks + [[0, 100, 120, 0, 900]]) == [11.0, 144.0, 10.0, 40.0]
    assert tl.phase_segments([]) is None
    t = tl.phase_table("gemm", marks)
    assert list(t["median_cycles"]) == tl.PHASES["gemm"]
    assert sum(t["median_cycles"].values()) == 205.0


def test_phase_names_cover_each_marked_kernel():
    # the attention kernel passes 3 marks (4 segments), the P.V kernel 4 (5)
    assert len(tl.PHASES["gemm"]) == 4
    assert len(tl.PHASES["attention"]) == 4
    assert len(tl.PHASES["attn_pv"]) == 5
    att = tl.phase_table("attention", [[100, 300, 400, 0, 1000]])
    assert att["median_cycles"] == dict(zip(tl.PHASES["attention"], [100.0, 200.0, 100.0, 600.0]))
    pv = tl.phase_table("attn_pv", [[100, 300, 400, 900, 1000]])
    assert pv["median_cycles"] == dict(zip(tl.PHASES["attn_pv"], [100.0, 200.0, 100.0, 500.0, 100.0]))
