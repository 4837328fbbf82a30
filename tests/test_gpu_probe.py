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
