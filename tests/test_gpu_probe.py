"""mvlm_probe_grid_barrier: the software grid-barrier probe behind the choice of
a graph of launches over a persistent single-launch decode step.  Each
protocol runs a few rounds with HBM idle and with HBM streaming; every wait is
bounded, so a round that cannot complete raises instead of hanging."""
from __future__ import annotations

import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("background", [False, True])
@pytest.mark.parametrize("variant", [0, 1, 2])
def test_grid_barrier_probe_runs(dev, variant, background):
    print(f"[barrier probe] variant={variant} background={background}", flush=True)
    us = dev.probe_grid_barrier(variant, 20, background)
    assert 0.1 < us < 1000.0, us


def test_grid_barrier_probe_rejects_bad_arguments(dev):
    import mvlm_amd as m
    with pytest.raises(m.native.MvlmError):
        dev.probe_grid_barrier(3, 10)
    with pytest.raises(m.native.MvlmError):
        dev.probe_grid_barrier(0, 0)


@pytest.mark.parametrize("variant,after", [(0, 0), (0, 9), (1, 0)])
def test_load_latency_probe_runs(dev, variant, after):
    """mvlm_probe_load_latency: per-wave first-load times at kernel start, ordered"""
    print(f"[latency probe] variant={variant} after={after}", flush=True)
    us = dev.probe_load_latency(variant, after)
    assert 0.0 <= us[0] <= us[1] <= us[2] <= us[3] < 1000.0, us


def test_load_latency_probe_rejects_bad_arguments(dev):
    import mvlm_amd as m
    with pytest.raises(m.native.MvlmError):
        dev.probe_load_latency(2, 0)
    with pytest.raises(m.native.MvlmError):
        dev.probe_load_latency(0, 3)
