import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

# The reference's error metric (tests/test_transformer_native.py:52-61): max
# |a-b| over max |ref|, with the fp32 tolerance RTOL = 1e-5 (:34-37).
RTOL = 1e-5

GOLDEN = os.path.join(ROOT, "tests", "golden")


def golden(name: str):
    return np.load(os.path.join(GOLDEN, name))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP path)")
    # A fresh checkout has no built libraries: build what is missing (the GPU
    # box receives them prebuilt and never compiles here).
    import subprocess
    if not os.path.exists(os.path.join(ROOT, "oracle", "libaero_cpuref.so")):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
    if not os.path.exists(os.path.join(ROOT, "aero_amd", "libaero_hip.so")):
        from aero_amd import build
        build.build()


def rel_to_scale(got, ref) -> float:
    got = np.asarray(got, np.float64).reshape(-1)
    ref = np.asarray(ref, np.float64).reshape(-1)
    assert got.shape == ref.shape, f"shape {got.shape} vs {ref.shape}"
    if ref.size == 0:
        return 0.0
    return float(np.abs(got - ref).max() / max(float(np.abs(ref).max()), 1e-30))


def bits_equal(a, b) -> bool:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.fixture(scope="session")
def hip():
    """The HIP library, on a machine with a GPU. Fails (never skips) when it is missing, so
    a GPU run cannot pass on a silent fallback."""
    from aero_amd import _lib

    reason = _lib.unavailable_reason()
    assert reason == "", f"HIP path unavailable on a GPU test run: {reason}"
    return _lib.lib()


@pytest.fixture(scope="session")
def oracle():
    from oracle import cpuref

    cpuref.lib()
    return cpuref
