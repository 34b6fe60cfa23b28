"""Peak-rate microbenchmarks on gfx950 (the reference's peak_compute_dpas
and peak_mem_2d programs): the MFMA checksum closed form and plausible
rates."""
import os
import re
import subprocess

import pytest

import xpu_playground_amd as xpu

pytestmark = pytest.mark.gpu


def run(*args):
    out = subprocess.run([os.path.join(xpu.BUILD_DIR, "peak"), *args], capture_output=True, text=True,
                         timeout=120)
    assert out.returncode == 0, out.stderr
    return out.stdout


def test_peak_compute_checksum_and_rate():
    # every MFMA adds 16 * 0.5 * 0.5 = 4 to each accumulator element:
    # sink = 28 + 8 chains * rounds * 4 (peak_compute_dpas.cpp:196-206)
    out = run("compute", "--rounds", "512", "--iterations", "5")
    assert "Checksum: PASS" in out
    tflops = float(re.search(r"Median BF16 compute: ([0-9.]+)", out).group(1))
    mhz = float(re.search(r"Shader clock during the loop: ([0-9.]+) MHz", out).group(1))
    print(out)
    assert 100.0 < tflops < 2600.0
    assert 500.0 < mhz < 3000.0


def test_peak_read_rate():
    out = run("mem", "--size-mib", "1024", "--iterations", "5")
    gbs = float(re.search(r"Median read bandwidth: ([0-9.]+)", out).group(1))
    print(out)
    assert 1000.0 < gbs < 9000.0


def test_handoff_probe_costs():
    # The test-only probe (tests/handoff_probe): a kernel boundary against
    # in-kernel all-to-all handoffs. Every variant completes its stages (the
    # waits are bounded) with the data it waited for.
    exe = os.path.join(os.path.dirname(os.path.abspath(__file__)), "handoff_probe", "build", "handoff_probe")
    out = subprocess.run([exe, "--launches", "200", "--stages", "100"], capture_output=True, text=True,
                         timeout=120)
    assert out.returncode == 0, out.stderr
    assert "Data check: PASS" in out.stdout
    m = re.search(r"Kernel boundary, \d+ blocks per launch: ([0-9.]+) us .* ([0-9.]+) us in a graph", out.stdout)
    assert m and 0 < float(m.group(2)) < 50
    costs = re.findall(r"In-kernel all-to-all handoff, .*: ([0-9.]+) us per stage", out.stdout)
    assert len(costs) == 4 and all(0 < float(c) < 1000 for c in costs)
    print(out.stdout)
