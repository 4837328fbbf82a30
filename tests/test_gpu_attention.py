"""Fused attention (mvlm_attention, mvlm_attention_prefill/_decode) against the
oracle's fp64 attention (oracle/oracle.c orc_attention_f64, the math of
attention.cl:46-179 and :197-295).

Tolerance per output element, with A = sum_k p_k |V_k| (the oracle's error
scale) and R = max_k scale sum_d |q_d k_d|:
  * probabilities are rounded to fp16 before the P V product: 2^-11 relative
    each, so at most 2^-11 A (taken as 2^-10 A for the fp32 rescaling steps);
  * fp32 score accumulation over head_dim terms: each score within
    head_dim 2^-24 R, which moves the weights by at most twice that, relative;
  * fp32 accumulation of P V over seq_kv terms: seq_kv 2^-24 A;
  * the output store: half an ulp of fp16 (or fp32).
The reference computes the same quantities in fp32 with native_exp and
native_rsqrt (approximate); the exact 1/sqrt(head_dim) is used here."""
from __future__ import annotations

import numpy as np
import pytest

import mvlm_amd as m
from mvlm_amd import native

pytestmark = pytest.mark.gpu

F16, F32 = m.F16, m.F32


def f16_bits(x):
    return np.asarray(x, np.float16).view(np.uint16)


def make_qkv(seq_q, seq_kv, H, D, seed, spread=1.0):
    rng = np.random.default_rng(seed)
    Q = f16_bits(rng.standard_normal((seq_q, H, D)) * spread)
    K = f16_bits(rng.standard_normal((seq_kv, H, D)) * spread)
    V = f16_bits(rng.standard_normal((seq_kv, H, D)))
    return Q, K, V


def download(O, o_dtype, n):
    if o_dtype == F32:
        return O.download(np.float32, n).astype(np.float64)
    return O.download(np.uint16, n).view(np.float16).astype(np.float64)


def check(got, O64, A, R, seq_kv, D, o_dtype):
    half_ulp = np.abs(O64) * (2.0 ** -11 if o_dtype == F16 else 2.0 ** -24) + (6e-8 if o_dtype == F16 else 0.0)
    tol = (2.0 ** -10 + seq_kv * 2.0 ** -24 + 2 * D * 2.0 ** -24 * R[..., None]) * A + half_ulp + 1e-12
    err = np.abs(got - O64)
    worst = float(np.max(err / tol))
    assert np.all(np.isfinite(got))
    assert np.all(err <= tol), worst
    return worst


def run(dev, orc, seq_q, seq_kv, H, D, causal, o_dtype, seed, scale=0.0, spread=1.0):
    Q, K, V = make_qkv(seq_q, seq_kv, H, D, seed, spread)
    dQ, dK, dV = dev.upload(Q), dev.upload(K), dev.upload(V)
    n = seq_q * H * D
    dO = dev.alloc(n * 4)
    print(f"[attention] seq_q={seq_q} seq_kv={seq_kv} heads={H} D={D} causal={causal} out={o_dtype}", flush=True)
    dev.attention(dQ, dK, dV, dO, o_dtype, seq_q, seq_kv, H, D, causal=causal, scale=scale)
    dev.sync()
    O64, A, R = orc.attention_f64(Q, K, V, seq_q, seq_kv, H, D, causal, scale if scale else 1.0 / np.sqrt(D))
    got = download(dO, o_dtype, n).reshape(seq_q, H, D)
    return check(got, O64, A, R, seq_kv, D, o_dtype)


@pytest.mark.parametrize("seq_q,seq_kv,H,D,causal,o_dtype", [
    (729, 729, 16, 72, False, F16),      # SigLIP layer: 729 patches, 16 heads of 72
    (729, 729, 16, 72, False, F32),
    (256, 256, 32, 64, True, F16),       # phi-1.5 prefill: 32 heads of 64
    (1, 300, 32, 64, False, F32),        # phi-1.5 decode against a 300-entry cache
    (33, 200, 4, 96, True, F32),         # chunked prefill: queries are the last 33 positions
    (5, 37, 3, 8, True, F32),
    (100, 100, 2, 128, True, F32),
    (31, 65, 7, 40, False, F16),
    (1, 1, 1, 8, False, F32),
    (64, 64, 1, 32, True, F16),
])
def test_attention_matches_oracle(dev, orc, seq_q, seq_kv, H, D, causal, o_dtype):
    run(dev, orc, seq_q, seq_kv, H, D, causal, o_dtype, seed=seq_q * 1000 + seq_kv + D)


def test_attention_explicit_scale_and_peaked_scores(dev, orc):
    # large scores (spread 3, scale 0.5) make the softmax nearly one-hot:
    # the running max must be rescaled correctly across key tiles
    run(dev, orc, 96, 160, 4, 64, False, F32, seed=7, scale=0.5, spread=3.0)
    run(dev, orc, 96, 160, 4, 64, True, F32, seed=8, scale=0.5, spread=3.0)


def test_attention_long_cache_decode(dev, orc):
    run(dev, orc, 1, 2048, 32, 64, False, F16, seed=9)
    run(dev, orc, 4, 2048, 32, 64, True, F32, seed=10)


@pytest.mark.parametrize("waves,splits", [("1", "5"), ("2", "5"), ("16", "5"), ("4", "2"), ("2", "1")])
def test_attention_forced_waves_with_key_splits(dev, orc, monkeypatch, waves, splits):
    """few (query tile, head) blocks: the keys split over workgroups (forced
    here; the automatic choice keeps short caches in one block) and merged by
    a second kernel; every waves-per-block and split variant must agree"""
    monkeypatch.setenv("MVLM_ATTN_WAVES", waves)
    monkeypatch.setenv("MVLM_ATTN_SPLITS", splits)
    run(dev, orc, 1, 700, 8, 64, False, F32, seed=41)
    run(dev, orc, 40, 300, 4, 72, True, F16, seed=42)


def test_attention_split_override_after_planning_is_refused(dev, monkeypatch):
    """a plan entry sized for one split (no workspace) must not launch with more
    splits when MVLM_ATTN_SPLITS changes afterwards: the launch is refused on
    the host"""
    from mvlm_amd import native
    H, D, S = 8, 64, 512
    q, k, v = dev.alloc(H * D * 2), dev.alloc(S * H * D * 2), dev.alloc(S * H * D * 2)
    o = dev.alloc(H * D * 4)
    monkeypatch.delenv("MVLM_ATTN_SPLITS", raising=False)
    plan = m.Plan(dev)
    plan.add_attention(q, k, v, o, F32, 1, S, H, D, causal=False)
    plan.run(1)
    dev.sync()
    monkeypatch.setenv("MVLM_ATTN_SPLITS", "4")
    with pytest.raises(native.MvlmError):
        plan.run(1)
    dev.sync()
    plan.destroy()


def test_attention_long_cache_single_block(dev, orc, monkeypatch):
    """a 2048-entry cache without key splits: 16 waves per (head) block, 4 key
    tiles each, merged in LDS"""
    monkeypatch.setenv("MVLM_ATTN_SPLITS", "1")
    run(dev, orc, 1, 2048, 32, 64, False, F16, seed=43)


def test_prefill_and_decode_entry_points(dev, orc):
    """the reference's dispatchers: prefill = causal, seq_q == seq_kv, fp16 out;
    decode = one query, no mask, fp16 out; both bit-identical to mvlm_attention"""
    S, H, D = 77, 8, 64
    Q, K, V = make_qkv(S, S, H, D, 21)
    dQ, dK, dV = dev.upload(Q), dev.upload(K), dev.upload(V)
    o1, o2 = dev.alloc(S * H * D * 2), dev.alloc(S * H * D * 2)
    dev.attention_prefill(dQ, dK, dV, o1, S, H, D)
    dev.attention(dQ, dK, dV, o2, F16, S, S, H, D, causal=True)
    dev.sync()
    assert np.array_equal(o1.download(np.uint16, S * H * D), o2.download(np.uint16, S * H * D))
    dq1 = dev.upload(Q[:1])
    dev.attention_decode(dq1, dK, dV, o1, S, H, D)
    dev.attention(dq1, dK, dV, o2, F16, 1, S, H, D, causal=False)
    dev.sync()
    a, b = o1.download(np.uint16, H * D), o2.download(np.uint16, H * D)
    assert np.array_equal(a, b)
    O64, A, R = orc.attention_f64(Q[:1], K, V, 1, S, H, D, False)
    check(a.view(np.float16).astype(np.float64).reshape(1, H, D), O64, A, R, S, D, F16)


def test_attention_in_plan_graph(dev, orc):
    S, H, D = 129, 16, 72
    Q, K, V = make_qkv(S, S, H, D, 31)
    dQ, dK, dV = dev.upload(Q), dev.upload(K), dev.upload(V)
    o1, o2 = dev.alloc(S * H * D * 4), dev.alloc(S * H * D * 4)
    dev.attention(dQ, dK, dV, o1, F32, S, S, H, D)
    plan = m.Plan(dev)
    plan.add_attention(dQ, dK, dV, o2, F32, S, S, H, D)
    plan.use_graph(True)
    for _ in range(3):
        plan.run(1)
        dev.sync()
        assert np.array_equal(o1.download(np.float32, S * H * D), o2.download(np.float32, S * H * D))
    plan.destroy()


def test_attention_argument_errors(dev):
    H, D, S = 2, 64, 16
    Q = dev.alloc(S * H * D * 2)
    O = dev.alloc(S * H * D * 4)

    def code(*a, **kw):
        with pytest.raises(m.MvlmError) as e:
            dev.attention(*a, **kw)
        return e.value.code
    assert code(Q, Q, Q, O, F16, S, S, H, 60) == native.ERR_UNSUPPORTED          # head_dim % 8
    assert code(Q, Q, Q, O, F16, 1, 1, 1, 136) == native.ERR_UNSUPPORTED         # head_dim > 128
    assert code(Q, Q, Q, O, F16, S + 1, S, H, D) == native.ERR_BUFFER_TOO_SMALL
    assert code(Q, Q, Q, O, m.BF16, S, S, H, D) == native.ERR_INVALID_ARG
    assert code(Q, Q, Q, O, F16, S, S - 1, H, D, causal=True) == native.ERR_INVALID_ARG
    assert code(Q, Q, Q, O, F16, S, S, H, D, scale=-1.0) == native.ERR_INVALID_ARG
    assert code(Q, Q, Q, O, F16, 0, S, H, D) == native.ERR_INVALID_ARG
