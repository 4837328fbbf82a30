"""On-device token pick (mvlm_argmax) against the oracle (oracle/oracle.c
orc_argmax, whose fp16 order equals the literal restatement of the
reference's host scan, moondream2.cpp:553-593).  Integer result: bit-exact."""
from __future__ import annotations

import numpy as np
import pytest

import mvlm_amd as m

pytestmark = pytest.mark.gpu


def bits_for(vals32, dt):
    if dt == m.F32:
        return np.ascontiguousarray(vals32, np.float32)
    if dt == m.F16:
        return np.asarray(vals32, np.float16).view(np.uint16)
    return (np.asarray(vals32, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def run(dev, orc, x, dt, rows, n, ld):
    dx = dev.upload(x)
    out = dev.alloc(rows * 4)
    print(f"[argmax] dtype={dt} rows={rows} n={n} ld={ld}", flush=True)
    dev.argmax(dx, dt, rows, n, ld, out)
    got = out.download(np.int32, rows)
    want = orc.argmax(x, dt, rows, n, ld)
    assert np.array_equal(got, want), (got[:8], want[:8])
    return got


@pytest.mark.parametrize("dt", [m.F32, m.F16, m.BF16])
@pytest.mark.parametrize("rows,n", [(1, 51200), (4, 51200), (16, 2048), (3, 1), (2, 1023), (1, 1 << 20)])
def test_argmax_random_rows(dev, orc, dt, rows, n):
    rng = np.random.default_rng(rows * 7 + n)
    x = bits_for(rng.standard_normal(rows * n) * 4, dt)
    run(dev, orc, x, dt, rows, n, n)


@pytest.mark.parametrize("dt", [m.F32, m.F16, m.BF16])
def test_argmax_ties_and_specials(dev, orc, dt):
    n = 51200
    rng = np.random.default_rng(5)
    base = rng.standard_normal((6, n)).astype(np.float32)
    base[0, [70, 9000, 51199]] = 100.0                  # tie across threads: first index wins
    base[1, :] = -np.inf                                 # all -inf: index 0
    base[2, [123, 40000]] = np.inf                       # two +inf
    base[3, 777] = np.nan                                # +NaN counts as +inf
    base[4, :] = 0.0
    base[4, 3333] = -0.0                                 # zeros all equal: index 0
    base[5, ::2] = 1.0                                   # every even index ties
    base[5, 1::2] = -1.0
    x = bits_for(base.ravel(), dt)
    got = run(dev, orc, x, dt, 6, n, n)
    assert got.tolist() == [70, 0, 123, 777, 0, 0]


@pytest.mark.parametrize("dt", [m.F32, m.F16, m.BF16])
def test_argmax_aligned_rows_with_tail(dev, orc, dt):
    """16-byte rows read in chunks, then n % (16 / size) trailing elements one at a time"""
    rows, n, ld = 3, 51197, 51200
    rng = np.random.default_rng(8)
    v = rng.standard_normal(rows * ld).astype(np.float32)
    v[n - 1] = 50.0                                      # row 0: the winner is a tail element
    v[ld + 7] = v[ld + n - 2] = 60.0                     # row 1: tie between a chunk and a tail element
    got = run(dev, orc, bits_for(v, dt), dt, rows, n, ld)
    assert got[0] == n - 1 and got[1] == 7


def test_argmax_f16_subnormals_and_stride(dev, orc):
    n, ld, rows = 4000, 4096, 3
    rng = np.random.default_rng(6)
    x = rng.integers(0, 1 << 16, rows * ld, dtype=np.uint16)
    x[:ld] = rng.integers(0, 0x400, ld, dtype=np.uint16) | (rng.integers(0, 2, ld, dtype=np.uint16) << 15)
    got = run(dev, orc, x, m.F16, rows, n, ld)
    assert got[0] == 0                                   # subnormals and zeros only: all keys equal
    for r in range(rows):
        assert got[r] == orc.lib().orc_argmax_f16_reference(np.ascontiguousarray(x[r * ld:r * ld + n]), n)


def test_argmax_after_lm_head_in_plan(dev, orc):
    """LM head (Q8_0 GEMV) then the token pick, captured in one graph."""
    N, K = 4096, 2048
    x = orc.normal_f32(K, 0x91)
    W = dev.pack(orc.q8_0_blocks(N * K // 32, 0x92), m.Q8_0, N, K)
    dx, logits, tok = dev.upload(x), dev.alloc(N * 4), dev.alloc(4)
    plan = m.Plan(dev)
    plan.add_gemv(dx, m.F32, W, logits, m.F32, 1)
    plan.add_argmax(logits, m.F32, 1, N, N, tok)
    plan.use_graph(True)
    for _ in range(3):
        plan.run(1)
        dev.sync()
        y = logits.download(np.float32, N)
        assert tok.download(np.int32, 1)[0] == orc.argmax(y, m.F32, 1, N, N)[0]
    plan.destroy()


def test_argmax_argument_errors(dev):
    x, out = dev.alloc(400), dev.alloc(4)
    for args in ((m.Q8_0, 1, 100, 100), (m.F32, 1, 100, 99), (m.F32, 0, 100, 100), (m.F32, 2, 100, 100)):
        with pytest.raises(m.MvlmError):
            dev.argmax(x, *args, out)
