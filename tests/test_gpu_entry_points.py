"""The reference's process-level entry points on gfx950: run_gemv
(gemv.cpp:157-170) and run_gemm (gemm.cpp:135-155) through the standalone
programs, the `peak gemv|gemm` launcher modes (peak_sycl.cpp:47-50) and an
in-process call of the exported C symbol, at the BASELINE shapes. Each run
must end with the reference's output contract (gemv.cpp:140-146,
gemm.cpp:121-127): Device / Type and shape / Median / Best /
Verification: PASS, and exit status 0."""
import ctypes
import os
import re
import subprocess

import pytest

import xpu_playground_amd as xpu

pytestmark = pytest.mark.gpu

NUM = r"([0-9]+\.[0-9]{2})"
GEMV_LINES = [r"^Device: .+$", r"^Type: (BF16|FP16), shape: (\d+)x(\d+)$",
              rf"^Median: {NUM} GFLOP/s, {NUM} GB/s$", rf"^Best:   {NUM} GFLOP/s, {NUM} GB/s$",
              r"^Verification: PASS$"]
GEMM_LINES = [r"^Device: .+$", r"^Type: (BF16|FP16), shape: (\d+)x(\d+)x(\d+)$", rf"^Median: {NUM} TFLOP/s$",
              rf"^Best:   {NUM} TFLOP/s$", r"^Verification: PASS$"]


def check_output(stdout, patterns):
    lines = stdout.splitlines()
    found = []
    for pat in patterns:
        hits = [re.match(pat, ln) for ln in lines]
        hits = [h for h in hits if h]
        assert len(hits) == 1, (pat, stdout)
        found.append(hits[0])
    # the reference's lines come in its order
    order = [lines.index(h.string) for h in found]
    assert order == sorted(order), stdout
    return found


def run(program, args, timeout=300):
    exe = [os.path.join(xpu.BUILD_DIR, program.split()[0])] + program.split()[1:] + args
    print("run:", " ".join(exe), flush=True)
    out = subprocess.run(exe, capture_output=True, text=True, timeout=timeout)
    assert out.returncode == 0, (out.returncode, out.stderr)
    return out.stdout


GEMV_CASES = [
    # BASELINE configs[0] and [1]: seeded U[-1,1] inputs
    (["--m", "4096", "--k", "4096", "--type", "bf16", "--init", "uniform"], "BF16", 4096, 4096),
    (["--size", "16384", "--type", "fp16", "--init", "uniform"], "FP16", 16384, 16384),
    # the reference's own hash initialisation (gemv.cpp:91-103, the default)
    (["--size", "4096", "--init", "reference"], "BF16", 4096, 4096),
    # ragged K (16-bit-load kernel) and a short matrix, hash and uniform
    (["--m", "1000", "--k", "1001", "--type", "fp16"], "FP16", 1000, 1001),
    (["--m", "1000", "--k", "1001", "--type", "fp16", "--init", "uniform"], "FP16", 1000, 1001),
    (["--m", "7", "--k", "64"], "BF16", 7, 64),
]


@pytest.mark.parametrize("args,type_,m,k", GEMV_CASES)
def test_run_gemv(args, type_, m, k):
    out = run("gemv", args + ["--iterations", "5", "--warmups", "2"])
    dev, shape, median, best, _ = check_output(out, GEMV_LINES)
    assert shape.groups() == (type_, str(m), str(k))
    gflops, gbs = float(median.group(1)), float(median.group(2))
    # the reference's accounting (gemv.cpp:109-110): 2MK FLOP and 2MK bytes
    assert gflops > 0 and abs(gbs - gflops) <= 0.011 * gflops + 0.02
    assert float(best.group(1)) >= gflops
    if m * k >= 4096 * 4096:
        assert gbs > 1000.0  # well above any host-memory path


GEMM_CASES = [
    (["--size", "4096", "--type", "bf16", "--init", "uniform"], "BF16", (4096, 4096, 4096)),  # configs[2]
    (["--m", "3000", "--n", "4097", "--k", "2050", "--type", "fp16", "--init", "uniform"], "FP16",
     (3000, 4097, 2050)),  # configs[3]
    (["--size", "4096", "--init", "constant"], "BF16", (4096, 4096, 4096)),    # gemm.cpp:81-85 KAT
    (["--m", "300", "--n", "200", "--k", "100", "--type", "fp16"], "FP16", (300, 200, 100)),
    (["--m", "33", "--n", "65", "--k", "17"], "BF16", (33, 65, 17)),
    (["--m", "33", "--n", "65", "--k", "17", "--init", "uniform"], "BF16", (33, 65, 17)),
]


@pytest.mark.parametrize("args,type_,shape", GEMM_CASES)
def test_run_gemm(args, type_, shape):
    out = run("gemm", args + ["--iterations", "3", "--warmups", "1"])
    dev, shp, median, best, _ = check_output(out, GEMM_LINES)
    assert shp.groups() == (type_,) + tuple(map(str, shape))
    # two decimals of TFLOP/s: a tiny product prints 0.00
    assert float(best.group(1)) >= float(median.group(1)) >= 0
    if shape == (4096, 4096, 4096):
        assert float(median.group(1)) > 200.0


def test_bare_programs_use_the_reference_inputs():
    # A caller that passes none of this build's extra flags gets the
    # reference's inputs and checks: gemv the hash initialisation of its
    # padded 16384^2 bf16 matrix (gemv.cpp:21,79-103), gemm the constant
    # A = 0.5, B = 0.25 at 4096^3 bf16 with the known answer 0.125 K = 512
    # (gemm.cpp:19,81-85,109-117), each with the reference's iteration counts.
    out = run("gemv", [])
    assert check_output(out, GEMV_LINES)[1].groups() == ("BF16", "16384", "16384")
    assert re.search(r"^Input: reference hash \(gemv.cpp:91-103\), row stride 16384$", out, re.M), out
    out = run("gemm", [])
    assert check_output(out, GEMM_LINES)[1].groups() == ("BF16", "4096", "4096", "4096")
    assert re.search(r"^Input: constant A = 0.5, B = 0.25 \(gemm.cpp:81-85\), expected 0.125 \* K = 512$", out,
                     re.M), out
    # the known-answer check, not the FP64 comparison of uniform inputs
    assert "Accuracy" not in out
    # a K that the reference pads: the hash runs over its 32-column row
    # stride, so every element carries the reference's value
    out = run("gemv", ["--m", "40", "--k", "1001", "--iterations", "2", "--warmups", "1"])
    assert re.search(r"^Input: reference hash .*row stride 1024$", out, re.M), out


def test_peak_launcher_gemv_and_gemm_modes():
    # peak_sycl.cpp:47-50: the mode selects the program, the rest are its flags
    out = run("peak gemv", ["--size", "16384", "--type", "fp16", "--iterations", "5", "--warmups", "2"])
    assert check_output(out, GEMV_LINES)[1].groups() == ("FP16", "16384", "16384")
    out = run("peak gemm", ["--size", "4096", "--iterations", "3", "--warmups", "1"])
    assert check_output(out, GEMM_LINES)[1].groups() == ("BF16", "4096", "4096", "4096")


def test_run_gemv_in_process(capfd):
    # the exported C symbol itself (the reference boundary: extern "C" run_gemv, gemv.cpp:157)
    lib = xpu.library()
    argv = [b"gemv", b"--m", b"2048", b"--k", b"3072", b"--type", b"fp16", b"--iterations", b"3",
            b"--warmups", b"1"]
    arr = (ctypes.c_char_p * len(argv))(*argv)
    rc = lib.run_gemv(len(argv), arr)
    out = capfd.readouterr().out
    assert rc == 0
    _, shape, _, _, _ = check_output(out, GEMV_LINES)
    assert shape.groups() == ("FP16", "2048", "3072")


def test_entry_points_report_errors_on_stderr():
    # an impossible allocation fails inside the run (not in flag parsing):
    # "Error: ..." on stderr and status 1 (gemv.cpp:163-168)
    exe = os.path.join(xpu.BUILD_DIR, "gemv")
    out = subprocess.run([exe, "--m", "4000000000", "--k", "4000000000"], capture_output=True, text=True,
                         timeout=120)
    assert out.returncode == 1 and out.stderr.startswith("Error: ")
    assert "Verification" not in out.stdout
