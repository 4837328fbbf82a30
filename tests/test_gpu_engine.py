"""The C++ mgpu:: drop-in (mvlm_amd/engine), exercised by tests/cpp/test_engine.cpp
the way the reference's gtest suites exercise src/engine (a device is required)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "mvlm_amd", "lib", "test_engine")


@pytest.mark.gpu
def test_cpp_engine_dropin():
    assert os.path.exists(EXE), "build first: python -m mvlm_amd.build"
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "PASSED" in r.stdout


def test_cpp_engine_skips_without_device():
    """Without a GPU the program reports a skip (exit 77), like GTEST_SKIP in test_device.cpp."""
    from mvlm_amd import native
    if native.device_count() > 0:
        pytest.skip("a GPU is visible")
    assert os.path.exists(EXE)
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=60)
    assert r.returncode == 77 and "SKIPPED" in r.stdout
