"""The decode fusion probe (tests/fusion_probe): its folded o_proj computes
the same layer as the shipped kernels, up to the re-association of the
o_proj sum, and its timing run produces every kernel of each sequence.
The probe's timings themselves are measurements, not asserted here."""
import os

import numpy as np
import pytest

import xpu_playground_amd as xpu
from fusion_probe import fusion_probe as fp

pytestmark = pytest.mark.gpu


def as_f32(codes):
    return (codes.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


@pytest.fixture(scope="module")
def probe_rt():
    assert os.path.exists(fp.MODULE), "build the probe first (__graft_entry__.build())"
    r = xpu.Runtime(module_path=fp.MODULE)
    yield r
    r.close()


@pytest.mark.parametrize("fold", [16, 8, 4])
@pytest.mark.parametrize("position", [0, 160, 255])
def test_fold_matches_the_shipped_layer(probe_rt, fold, position):
    print(f"fusion probe check: fold{fold} at position {position}", flush=True)
    out = fp.check_layer(probe_rt, position, fold)
    xb, hb = (as_f32(a) for a in out["base"])
    xf, hf = (as_f32(a) for a in out[f"fold{fold}"])
    assert np.all(np.isfinite(xb)) and np.all(np.isfinite(hb))
    # x + o after o_proj: equal, or one bf16 step of the larger magnitude
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.maximum(np.abs(xb), np.abs(xf)), 1e-30))) - 7)
    assert np.all(np.abs(xb - xf) <= ulp), np.argwhere(np.abs(xb - xf) > ulp)[:5]
    assert np.mean(xb != xf) <= 0.05
    # the [gate; up] + SiLU output on those inputs
    rel = np.linalg.norm(hb - hf) / np.linalg.norm(hb)
    print(f"x codes differing {np.mean(xb != xf):.4f}, h rel-L2 {rel:.2e}", flush=True)
    assert rel <= 1e-2


def test_timing_run_covers_each_sequence(probe_rt):
    st = fp.tl.Stamps(probe_rt)
    m = fp.Model(probe_rt, 160, layers=4)
    try:
        for variant, kernels in (("base", {"qkv", "attention", "o_proj", "gate_up", "down"}),
                                 ("fold16", {"qkv", "attention", "gate_up", "down"})):
            print(f"fusion probe timing: {variant}", flush=True)
            r = fp.time_variant(m, st, variant, reps=3)
            assert set(r["per_kernel"]) == kernels
            # one launch per layer; the timestamp grouping (a new launch where
            # a wave enters after every earlier wave has left) can split a
            # launch whose last blocks start late, which counts it twice
            assert all(4 <= v["launches_per_token"] <= 4.5 for v in r["per_kernel"].values()), r["per_kernel"]
            assert r["us_per_token_layers"] > 0
    finally:
        m.close()
