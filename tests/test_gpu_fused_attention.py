"""Plan fusion: a decode attention (one query per head against a KV cache,
attention_decode in attention.cl:197-295) carried by the grouped GEMV launch
that reads its output (the output projection after it, moondream2.cpp:423-446).

Checked on the GPU through the C ABI, after every graph replay:
  * the attention output o against the oracle's fp64 attention, within the
    tolerance of the attention tests (2^-10 A + seq_kv 2^-24 A + 2 D 2^-24 R A
    + half an fp32 ulp, A = sum_k p_k |V_k|, R = max_k scale sum_d |q_d k_d|);
  * the entry reading o as x against the oracle's fp32 GEMV on the o the GPU
    produced (1e-5 S, S = sum_k |x_k w_k|), the other entry bit-identical to
    the same plan run unfused, whose o (the matrix-core attention kernel)
    meets the same bound;
  * plan.check(): no wait gave up.
Every replay must give the same bits: the counters the launch hands work
through return to zero by its end."""
from __future__ import annotations

import numpy as np
import pytest

import mvlm_amd as m

pytestmark = pytest.mark.gpu

F16, F32 = m.F16, m.F32


def f16_bits(x):
    return np.asarray(x, np.float16).view(np.uint16)


def attention_tol(O64, A, R, seq_kv, D):
    return (2.0 ** -10 + seq_kv * 2.0 ** -24 + 2 * D * 2.0 ** -24 * R[..., None]) * A + np.abs(O64) * 2.0 ** -24 + 1e-12


def gemv_check(orc, x, W, y, rows, scratch):
    deq = W.dequant_rows(rows, scratch).astype(np.float32)
    K = x.size
    ref = orc.gemm_nk("f32", np.ascontiguousarray(x.reshape(1, K)), np.ascontiguousarray(deq), 1, len(rows), K)
    _, S = orc.gemm_f64(x.reshape(1, K).astype(np.float64), deq.astype(np.float64), 1, len(rows), K)
    err = np.abs(y[rows].astype(np.float64) - ref.reshape(-1))
    assert np.all(err <= 1e-5 * S.reshape(-1)), float(np.max(err / (1e-5 * S.reshape(-1))))


class Case:
    """attention (q, K, V -> o) then grouped {o -> W1 -> y1, x2 -> W2 -> y2}"""

    def __init__(self, dev, wdt, T, H, D, N1, N2, K2, seed):
        rng = np.random.default_rng(seed)
        self.T, self.H, self.D = T, H, D
        self.q = f16_bits(rng.standard_normal((H, D)))
        self.k = f16_bits(rng.standard_normal((T, H, D)))
        self.v = f16_bits(rng.standard_normal((T, H, D)))
        self.dq, self.dk, self.dv = dev.upload(self.q), dev.upload(self.k), dev.upload(self.v)
        self.o = dev.alloc(H * D * 4)
        self.W1 = dev.random_weight(wdt, N1, H * D, seed ^ 0x51, 0.02)
        self.W2 = dev.random_weight(wdt, N2, K2, seed ^ 0x52, 0.02)
        self.x2 = dev.fill_normal(dev.alloc(K2 * 4), F32, K2, seed ^ 0x53, 1.0)
        self.y1, self.y2 = dev.alloc(N1 * 4), dev.alloc(N2 * 4)
        self.N1, self.N2, self.K2 = N1, N2, K2
        self.scratch = dev.alloc(max(N1 * H * D, N2 * K2) * 4)

    def plan(self, dev, fuse=True, bias=None):
        p = m.Plan(dev)
        p.add_attention(self.dq, self.dk, self.dv, self.o, F32, 1, self.T, self.H, self.D)
        eps = None if bias is None else [{"bias": bias}, None]
        p.add_gemv_grouped([(self.o, F32, self.W1, self.y1, F32), (self.x2, F32, self.W2, self.y2, F32)],
                           epilogues=eps)
        p.set_fusion(fuse)
        return p

    def outputs(self):
        return (self.o.download(np.float32, self.H * self.D), self.y1.download(np.float32, self.N1),
                self.y2.download(np.float32, self.N2))

    def check_attention(self, orc, o):
        O64, A, R = orc.attention_f64(self.q[None], self.k, self.v, 1, self.T, self.H, self.D, False,
                                      1.0 / np.sqrt(self.D))
        got = o.astype(np.float64).reshape(1, self.H, self.D)
        tol = attention_tol(O64, A, R, self.T, self.D)
        err = np.abs(got - O64)
        assert np.all(np.isfinite(got))
        assert np.all(err <= tol), float(np.max(err / tol))

    def free(self):
        self.W1.free()
        self.W2.free()


def run_case(dev, orc, wdt, T, H, D, N1=2048, N2=2048, K2=8192, seed=7, replays=4):
    print(f"[fused attention] wdt={wdt} T={T} H={H} D={D} N1={N1} N2={N2} K2={K2}", flush=True)
    c = Case(dev, wdt, T, H, D, N1, N2, K2, seed)
    ref = c.plan(dev, fuse=False)
    assert ref.fused() == 0
    ref.run(1)
    ref.check()
    o_ref, y1_ref, y2_ref = c.outputs()
    fused = c.plan(dev, fuse=True)
    assert fused.fused() == 1
    fused.use_graph(True)
    first = None
    for r in range(replays):
        for b in (c.o, c.y1, c.y2):
            b.zero()
        fused.run(1)
        fused.check()
        o, y1, y2 = c.outputs()
        if first is None:
            first = (o, y1, y2)
            c.check_attention(orc, o)
            rows = np.unique(np.linspace(0, N1 - 1, 128).astype(np.int64))
            gemv_check(orc, o, c.W1, y1, rows, c.scratch)
            assert np.array_equal(y2, y2_ref)
            c.check_attention(orc, o_ref)
        else:
            for a, b in zip(first, (o, y1, y2)):
                assert np.array_equal(a, b), r
    fused.destroy()
    ref.destroy()
    c.free()


@pytest.mark.parametrize("T", [1, 5, 127, 300, 512, 2048, 4100])
def test_fused_decode_attention_q8_0(dev, orc, T):
    run_case(dev, orc, m.Q8_0, T, 32, 64)


@pytest.mark.parametrize("wdt,T,H,D", [
    (m.Q4_0, 512, 32, 64),       # Phi-1.5 shapes, Q4_0 weights
    (m.Q4_0, 2048, 32, 64),
    (m.F32, 200, 16, 64),        # dense fp32 weights (rows of 4 KiB)
    (m.F16, 300, 32, 64),
    (m.Q8_0, 700, 16, 128),      # head_dim 128
    (m.Q8_0, 9, 3, 64),          # few heads: many splits per head
    (m.Q4_0, 3000, 5, 128),
])
def test_fused_decode_attention_shapes(dev, orc, wdt, T, H, D):
    run_case(dev, orc, wdt, T, H, D, N1=1000, N2=3000, K2=2048)


def test_fused_with_epilogue_and_plan_profile(dev, orc):
    c = Case(dev, m.Q8_0, 512, 32, 64, 2048, 2048, 8192, 11)
    bias = dev.fill_normal(dev.alloc(2048 * 4), F32, 2048, 0x77, 0.5)
    p = c.plan(dev, fuse=True, bias=bias)
    assert p.fused() == 1
    p.run(2)
    p.check()
    o, y1, _ = c.outputs()
    c.check_attention(orc, o)
    rows = np.arange(0, 2048, 16)
    deq = c.W1.dequant_rows(rows, c.scratch)
    _, S = orc.gemm_f64(o.reshape(1, -1).astype(np.float64), deq.astype(np.float64), 1, len(rows), 2048)
    want = deq.astype(np.float64) @ o.astype(np.float64) + bias.download(np.float32, 2048)[rows]
    assert np.all(np.abs(y1[rows] - want) <= 1.2e-5 * S.reshape(-1) + 1e-6 * np.abs(want))
    ms = p.profile()
    assert ms[0] == 0.0 and ms[1] > 0.0       # the attention is timed with the launch carrying it
    p.check()
    p.destroy()
    c.free()


def test_fusion_is_refused_where_it_does_not_fit(dev):
    H, D, T = 32, 64, 64
    rng = np.random.default_rng(3)
    q = dev.upload(f16_bits(rng.standard_normal((2, H, D))))
    k = dev.upload(f16_bits(rng.standard_normal((T, H, D))))
    v = dev.upload(f16_bits(rng.standard_normal((T, H, D))))
    o32, o16 = dev.alloc(2 * H * D * 4), dev.alloc(H * D * 2)
    W = dev.random_weight(m.Q8_0, 512, H * D, 5, 0.02)
    Wlong = dev.random_weight(m.Q8_0, 512, 4096, 6, 0.02)
    x = dev.fill_normal(dev.alloc(4096 * 4), F32, 4096, 9, 1.0)
    y = dev.alloc(512 * 4)

    def pair(o, o_dtype, seq_q, entries, between=False):
        p = m.Plan(dev)
        p.add_attention(q, k, v, o, o_dtype, seq_q, T, H, D)
        if between:
            p.add_gemv(x, F32, Wlong, y, F32)
        p.add_gemv_grouped(entries)
        n = p.fused()
        p.destroy()
        return n

    assert pair(o32, F32, 1, [(o32, F32, W, y, F32)]) == 1
    assert pair(o32, F32, 2, [(o32, F32, W, y, F32)]) == 0          # more than one query
    assert pair(o32, F32, 1, [(x, F32, W, y, F32)]) == 0            # nothing reads o
    assert pair(o32, F32, 1, [(o32, F32, W, y, F32)], between=True) == 0
    assert pair(o32, F32, 1, [(o32, F32, W, q, F32)]) == 0          # an entry writes q
    assert pair(o32, F32, 1, [(o32, F32, W, o32, F32)]) == 0        # an entry writes o
    # an F16 output read as the F16 x of dense F16 weights
    W16 = dev.pack(f16_bits(rng.standard_normal((512, H * D)) * 0.02), F16, 512, H * D)
    p = m.Plan(dev)
    p.add_attention(q, k, v, o16, F16, 1, T, H, D)
    p.add_gemv_grouped([(o16, F16, W16, y, F32)])
    assert p.fused() == 0
    p.destroy()
    W.free()
    Wlong.free()
    W16.free()


def test_long_rows_reading_o_are_not_fused(dev):
    H, D, T = 64, 128, 100          # o has 8192 values: Q8_0 rows of 8 KiB of codes
    rng = np.random.default_rng(4)
    q = dev.upload(f16_bits(rng.standard_normal((H, D))))
    k = dev.upload(f16_bits(rng.standard_normal((T, H, D))))
    v = dev.upload(f16_bits(rng.standard_normal((T, H, D))))
    o = dev.alloc(H * D * 4)
    W = dev.random_weight(m.Q8_0, 256, H * D, 8, 0.02)
    y = dev.alloc(256 * 4)
    p = m.Plan(dev)
    p.add_attention(q, k, v, o, F32, 1, T, H, D)
    p.add_gemv_grouped([(o, F32, W, y, F32)])
    assert p.fused() == 0
    p.run(1)
    p.check()
    p.destroy()
    W.free()


# ---- decode attention step: q, k, v from a fused QKV projection's output -----

def f16_round(x):
    return np.asarray(x, np.float32).astype(np.float16)


class StepCase:
    """group {x -> Wqkv -> qkv (N = 3 H D), x2 -> W2 -> y2}, then the decode step
    (qkv, caches with `cached` rows + 1, o)"""

    def __init__(self, dev, wdt, T, H, D, K, N2, K2, seed):
        rng = np.random.default_rng(seed)
        self.T, self.H, self.D, self.K = T, H, D, K
        HD = H * D
        self.Wqkv = dev.random_weight(wdt, 3 * HD, K, seed ^ 0x61, 0.05)
        self.W2 = dev.random_weight(wdt, N2, K2, seed ^ 0x62, 0.02)
        self.x = dev.fill_normal(dev.alloc(K * 4), F32, K, seed ^ 0x63, 1.0)
        self.x2 = dev.fill_normal(dev.alloc(K2 * 4), F32, K2, seed ^ 0x64, 1.0)
        self.qkv = dev.alloc(3 * HD * 4)
        self.y2 = dev.alloc(N2 * 4)
        self.k0 = f16_bits(rng.standard_normal((T + 1, H, D)))
        self.v0 = f16_bits(rng.standard_normal((T + 1, H, D)))
        self.kc, self.vc = dev.upload(self.k0), dev.upload(self.v0)
        self.o = dev.alloc(HD * 4)
        self.N2, self.K2 = N2, K2
        self.scratch = dev.alloc(max(3 * HD * K, N2 * K2) * 4)

    def plan(self, dev, fuse=True):
        p = m.Plan(dev)
        p.set_fusion(fuse)
        p.add_gemv_grouped([(self.x, F32, self.Wqkv, self.qkv, F32), (self.x2, F32, self.W2, self.y2, F32)])
        p.add_attention_decode_step(self.qkv, self.kc, self.vc, self.o, self.T, self.H, self.D)
        return p

    def reset_caches(self):
        self.kc.upload(self.k0)
        self.vc.upload(self.v0)

    def check(self, orc, o, qkv):
        H, D, T = self.H, self.D, self.T
        HD = H * D
        q = f16_bits(qkv[:HD].reshape(1, H, D))
        kn, vn = f16_bits(qkv[HD:2 * HD].reshape(H, D)), f16_bits(qkv[2 * HD:].reshape(H, D))
        kc = self.kc.download(np.uint16, (T + 1) * HD).reshape(T + 1, H, D)
        vc = self.vc.download(np.uint16, (T + 1) * HD).reshape(T + 1, H, D)
        assert np.array_equal(kc[T], kn) and np.array_equal(vc[T], vn)          # the append, RNE fp16
        assert np.array_equal(kc[:T], self.k0[:T]) and np.array_equal(vc[:T], self.v0[:T])
        O64, A, R = orc.attention_f64(q, kc, vc, 1, T + 1, H, D, False, 1.0 / np.sqrt(D))
        got = o.astype(np.float64).reshape(1, H, D)
        tol = attention_tol(O64, A, R, T + 1, D)
        assert np.all(np.isfinite(got))
        assert np.all(np.abs(got - O64) <= tol), float(np.max(np.abs(got - O64) / tol))

    def free(self):
        self.Wqkv.free()
        self.W2.free()


@pytest.mark.parametrize("T,H,D", [(0, 32, 64), (1, 32, 64), (100, 32, 64), (512, 32, 64), (2047, 32, 64),
                                   (300, 16, 128), (33, 5, 64)])
def test_attention_decode_step_direct(dev, orc, T, H, D):
    print(f"[decode step] direct T={T} H={H} D={D}", flush=True)
    rng = np.random.default_rng(T + H)
    HD = H * D
    qkv = rng.standard_normal(3 * HD).astype(np.float32)
    k0 = f16_bits(rng.standard_normal((T + 1, H, D)))
    v0 = f16_bits(rng.standard_normal((T + 1, H, D)))
    dq, kc, vc, o = dev.upload(qkv), dev.upload(k0), dev.upload(v0), dev.alloc(HD * 4)
    dev.attention_decode_step(dq, kc, vc, o, T, H, D)
    dev.sync()
    c = StepCase.__new__(StepCase)
    c.T, c.H, c.D, c.kc, c.vc, c.k0, c.v0 = T, H, D, kc, vc, k0, v0
    c.check(orc, o.download(np.float32, HD), qkv)


@pytest.mark.parametrize("wdt,T,H,D,K", [(m.Q8_0, 512, 32, 64, 2048), (m.Q8_0, 2048, 32, 64, 2048),
                                         (m.Q4_0, 512, 32, 64, 2048), (m.Q8_0, 0, 32, 64, 2048),
                                         (m.Q8_0, 300, 16, 128, 1024), (m.F32, 77, 5, 64, 256)])
def test_fused_decode_step(dev, orc, wdt, T, H, D, K):
    print(f"[decode step] fused wdt={wdt} T={T} H={H} D={D} K={K}", flush=True)
    c = StepCase(dev, wdt, T, H, D, K, 3000, 2048, 17)
    ref = c.plan(dev, fuse=False)
    assert ref.fused() == 0
    ref.run(1)
    ref.check()
    o_ref, y2_ref = c.o.download(np.float32, H * D), c.y2.download(np.float32, c.N2)
    qkv_ref = c.qkv.download(np.float32, 3 * H * D)
    c.check(orc, o_ref, qkv_ref)
    fused = c.plan(dev, fuse=True)
    assert fused.fused() == 1
    fused.use_graph(True)
    first = None
    for r in range(4):
        c.reset_caches()
        for b in (c.o, c.qkv, c.y2):
            b.zero()
        fused.run(1)
        fused.check()
        got = (c.o.download(np.float32, H * D), c.qkv.download(np.float32, 3 * H * D),
               c.y2.download(np.float32, c.N2))
        if first is None:
            first = got
            assert np.array_equal(got[1], qkv_ref) and np.array_equal(got[2], y2_ref)
            c.check(orc, got[0], got[1])
            rows = np.unique(np.linspace(0, 3 * H * D - 1, 128).astype(np.int64))
            gemv_check(orc, c.x.download(np.float32, K), c.Wqkv, got[1], rows, c.scratch)
        else:
            for a, b in zip(first, got):
                assert np.array_equal(a, b), r
    fused.destroy()
    ref.destroy()
    c.free()


def test_decode_step_not_fused_when_it_does_not_fit(dev):
    c = StepCase(dev, m.Q8_0, 64, 32, 64, 2048, 512, 2048, 5)
    # the other entry reads the cache: not fused
    p = m.Plan(dev)
    p.add_gemv_grouped([(c.x, F32, c.Wqkv, c.qkv, F32), (c.kc, F32, c.W2, c.y2, F32)])
    p.add_attention_decode_step(c.qkv, c.kc, c.vc, c.o, c.T, c.H, c.D)
    assert p.fused() == 0
    p.destroy()
    # no entry writes qkv
    p = m.Plan(dev)
    p.add_gemv_grouped([(c.x2, F32, c.W2, c.y2, F32)])
    p.add_attention_decode_step(c.qkv, c.kc, c.vc, c.o, c.T, c.H, c.D)
    assert p.fused() == 0
    p.destroy()
    # an entry writes o
    p = m.Plan(dev)
    p.add_gemv_grouped([(c.x, F32, c.Wqkv, c.qkv, F32), (c.x2, F32, c.W2, c.o, F32)])
    p.add_attention_decode_step(c.qkv, c.kc, c.vc, c.o, c.T, c.H, c.D)
    assert p.fused() == 0
    p.destroy()
    c.free()


def test_decode_step_carried_by_the_readers_launch(dev, orc):
    """group A writes qkv, the step, group B reads o: the step runs in B's launch
    (A's launch stays plain), every replay equal, o and B's reader against the
    oracle"""
    c = StepCase(dev, m.Q8_0, 512, 32, 64, 2048, 2048, 8192, 23)
    W3 = dev.random_weight(m.Q8_0, 2048, 2048, 0x91, 0.02)
    y3 = dev.alloc(2048 * 4)

    def plan(fuse):
        p = m.Plan(dev)
        p.set_fusion(fuse)
        p.add_gemv_grouped([(c.x, F32, c.Wqkv, c.qkv, F32), (c.x2, F32, c.W2, c.y2, F32)])
        p.add_attention_decode_step(c.qkv, c.kc, c.vc, c.o, c.T, c.H, c.D)
        p.add_gemv_grouped([(c.o, F32, W3, y3, F32), (c.x2, F32, c.W2, c.y2, F32)])
        return p

    ref = plan(False)
    ref.run(1)
    ref.check()
    y3_ref = y3.download(np.float32, 2048)
    p = plan(True)
    assert p.fused() == 1
    ms = p.profile()
    assert ms[0] > 0 and ms[1] == 0 and ms[2] > 0       # the step is timed with B's launch
    p.use_graph(True)
    first = None
    for r in range(4):
        c.reset_caches()
        for b in (c.o, c.qkv, y3):
            b.zero()
        p.run(1)
        p.check()
        got = (c.o.download(np.float32, 2048), c.qkv.download(np.float32, 6144), y3.download(np.float32, 2048))
        if first is None:
            first = got
            c.check(orc, got[0], got[1])
            rows = np.unique(np.linspace(0, 2047, 128).astype(np.int64))
            gemv_check(orc, got[0], W3, got[2], rows, c.scratch)
            assert np.allclose(got[2], y3_ref, rtol=1e-4, atol=1e-4)
        else:
            for a, b in zip(first, got):
                assert np.array_equal(a, b), r
    p.destroy()
    ref.destroy()
    W3.free()
    c.free()


def test_wait_give_up_is_reported_and_the_next_run_is_exact(dev, orc, monkeypatch):
    """The give-up path of the bounded wait, forced from the host: with a wait
    bound of 0 ticks (MVLM_ATTN_WAIT_TICKS, read at every launch of an eager
    plan) a reader of o that polls before the attention is done gives up at
    once; it stores NaN instead of its rows and sets the site's error word.
    Every kernel still ends normally.  plan.check() reports the give-up and
    clears the site's counters, and the next run with the normal bound is
    bit-identical to the unfused plan's where it does not read o and within
    tolerance where it does."""
    c = Case(dev, m.Q8_0, 2048, 32, 64, 2048, 2048, 8192, 13)
    ref = c.plan(dev, fuse=False)
    ref.run(1)
    ref.check()
    o_ref, y1_ref, y2_ref = c.outputs()
    p = c.plan(dev, fuse=True)
    assert p.fused() == 1
    monkeypatch.setenv("MVLM_ATTN_WAIT_TICKS", "0")
    gave_up = 0
    for r in range(5):
        print(f"[give-up] forced run {r}", flush=True)
        for b in (c.o, c.y1, c.y2):
            b.zero()
        p.run(1)
        try:
            p.check()
        except m.native.MvlmError:
            gave_up += 1
            _, y1, y2 = c.outputs()
            assert np.isnan(y1).any()                # the readers that gave up stored NaN
            assert np.array_equal(y2, y2_ref)        # the rows that do not read o are untouched by it
    assert gave_up > 0
    monkeypatch.delenv("MVLM_ATTN_WAIT_TICKS")
    for r in range(3):
        print(f"[give-up] normal run {r}", flush=True)
        for b in (c.o, c.y1, c.y2):
            b.zero()
        p.run(1)
        p.check()
        o, y1, y2 = c.outputs()
        c.check_attention(orc, o)
        assert np.all(np.isfinite(y1))
        rows = np.unique(np.linspace(0, 2047, 128).astype(np.int64))
        gemv_check(orc, o, c.W1, y1, rows, c.scratch)
        assert np.array_equal(y2, y2_ref)
    p.destroy()
    ref.destroy()
    c.free()
