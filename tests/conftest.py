import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
os.environ.setdefault("MVLM_QUIET", "1")   # error paths are exercised on purpose


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle_ffi
    oracle_ffi.lib()
    return oracle_ffi


@pytest.fixture(scope="session")
def dev():
    """The GPU under test.  Fails (does not skip) when the HIP library or the
    device is missing: a GPU test must never pass without the native path."""
    import mvlm_amd
    d = mvlm_amd.Device(0)
    info = d.info()
    print(f"\n[device] {info.device_name.decode()} {info.arch_name.decode()} "
          f"CUs={info.compute_units} clock={info.max_clock_mhz} MHz", flush=True)
    yield d
    d.close()


def within(y, ref, scale, rtol, extra=0.0):
    """|y - ref| <= rtol * scale + extra, elementwise; returns (ok, worst ratio)."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(y - ref)
    bound = rtol * np.asarray(scale, np.float64) + extra
    ratio = float(np.max(err / np.maximum(bound, 1e-300))) if err.size else 0.0
    return bool(np.all(err <= bound)), ratio
