import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, REPO)
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 (MI355X) GPU; runs the HIP kernels")


@pytest.fixture(scope="session")
def rt():
    """One runtime (device, stream, code object) for all GPU tests."""
    import xpu_playground_amd as xpu

    runtime = xpu.Runtime()
    assert runtime.arch.startswith("gfx950"), runtime.arch
    print(f"\n[gpu] {runtime.device_name} {runtime.arch} {runtime.compute_units} CUs", flush=True)
    yield runtime
    runtime.close()
