"""The decode-step plans bench.py times, checked end to end on the GPU.

bench.build_decode_plan and bench.build_token_plan are the exact plans of the
benchmark's headline step (Phi-1.5, 24 layers of {QKV 2048->6144, dense
2048->2048, fc1 2048->8192, fc2 8192->2048} + LM head 2048->51200, grouped
into 49 launches, replayed as a HIP graph; moondream2.cpp:359-541 is the
reference's sequence of these projections).  After graph replays every one of
the 97 outputs is compared with the oracle's fp32 GEMV (exact dequantization,
fp32 fma chain in ascending k) on 256 rows spread over the output, within
1e-5 * S (S = sum_k |x_k w_k|); the token pick at the end of the decode-token
plan must be the oracle's argmax of the LM head's logits."""
from __future__ import annotations

import numpy as np
import pytest

import bench
import mvlm_amd as m

pytestmark = pytest.mark.gpu

ROWS = 256


def sample_rows(N):
    return np.unique(np.linspace(0, N - 1, ROWS).astype(np.int64))


def check_outputs(dev, orc, weights, io, M):
    """every GEMV output (sampled rows) against the oracle; with io["ep"], the
    output is the epilogue (bias, GELU, residual) applied in fp64 to the fp64
    product, within the accumulator bound carried through it plus fp32 ulps"""
    scratch = dev.alloc(max(N * K for _, N, K in bench.PHI_STEP) * 4)
    if isinstance(io["x"], dict):   # one input per projection name
        xs = {name: io["x"][name].download(np.float32, M * K).reshape(M, K) for name, _, K in bench.PHI_STEP[:4]}
        x_of = [xs["qkv" if name == "lm_head" else name] for name, _, _ in bench.PHI_STEP]
    else:                           # one input per GEMV (the outputs of earlier stages)
        x_of = [x.download(np.float32, M * K).reshape(M, K) for x, (_, _, K) in zip(io["x"], bench.PHI_STEP)]
        xs = x_of
    eps = io.get("ep") or [None] * len(bench.PHI_STEP)
    for i, ((name, N, K), W, y, ep) in enumerate(zip(bench.PHI_STEP, weights, io["y"], eps)):
        x = x_of[i]
        rows = sample_rows(N)
        deq = W.dequant_rows(rows, scratch)                          # [rows, K] fp32, exact
        got = y.download(np.float32, M * N).reshape(M, N)[:, rows].astype(np.float64)
        if ep is None:
            ref = orc.gemm_nk("f32", np.ascontiguousarray(x), np.ascontiguousarray(deq), M, len(rows), K)
            _, S = orc.gemm_f64(x.astype(np.float64), deq.astype(np.float64), M, len(rows), K)
            err = np.abs(got - ref.reshape(M, len(rows)))
            assert np.all(err <= 1e-5 * S), (i, name, float(np.max(err / (1e-5 * S))))
            continue
        Y64, S = orc.gemm_f64(x.astype(np.float64), deq.astype(np.float64), M, len(rows), K)
        bias = ep["bias"].download(np.float32, N)[rows].astype(np.float64) if ep.get("bias") else None
        res = (ep["residual"].download(np.float32, M * N).reshape(M, N)[:, rows].astype(np.float64)
               if ep.get("residual") else None)
        act = ep.get("act", 0)
        ref = orc.epilogue_f64(Y64, bias, None, res, act)
        body = orc.epilogue_f64(Y64, bias, act=act)
        tol = 1e-5 * S * 1.2 + 4e-6 * (np.abs(body) + (np.abs(res) if res is not None else 0.0)) + 1e-30
        err = np.abs(got - ref)
        assert np.all(err <= tol), (i, name, float(np.max(err / tol)))
    return xs


@pytest.mark.parametrize("qt,M", [("q8_0", 1), ("q4_0", 1), ("q4_0", 2), ("q8_0", 3), ("q4_0", 4), ("q8_0", 4),
                                  ("q8_0", 9), ("q4_0", 16), ("q8_0", 16)])
def test_decode_step_plan_outputs(dev, orc, qt, M):
    print(f"[decode plan] {qt} M={M}", flush=True)
    plan, weights, grouped, io = bench.build_decode_plan(dev, m, qt, M, True)
    assert grouped and len(plan) == 49
    for y in io["y"]:
        y.zero()
    plan.use_graph(True)
    plan.run(3)
    dev.sync()
    check_outputs(dev, orc, weights, io, M)
    plan.destroy()
    for W in weights:
        W.free()


@pytest.mark.parametrize("qt,cache,fuse", [("q8_0", 512, True), ("q8_0", 512, False), ("q4_0", 2048, True)])
def test_decode_token_plan_picks_the_argmax(dev, orc, qt, cache, fuse):
    """The token plan end to end: every GEMV output (dense on the attention
    output the plan computed), the attention step of the first and last layer
    (the cache append bit for bit, the output against the oracle's fp64
    attention over cache + 1 keys, the attention tests' bound), and the token
    pick."""
    print(f"[token plan] {qt} cache {cache} fuse={fuse}", flush=True)
    plan, weights, io = bench.build_token_plan(dev, m, qt, cache, fuse)
    assert len(plan) == 24 * 3 + 2
    assert plan.fused() == (24 if fuse else 0)
    plan.use_graph(True)
    plan.run(2)
    plan.check()
    check_outputs(dev, orc, weights, io, 1)
    H, D = 32, 64
    HD = H * D
    for layer in (0, 23):
        qkv = io["y"][4 * layer].download(np.float32, 3 * HD)
        q = np.asarray(qkv[:HD], np.float16).view(np.uint16).reshape(1, H, D)
        kc = io["kc"][layer].download(np.uint16, (cache + 1) * HD).reshape(cache + 1, H, D)
        vc = io["vc"][layer].download(np.uint16, (cache + 1) * HD).reshape(cache + 1, H, D)
        assert np.array_equal(kc[cache], np.asarray(qkv[HD:2 * HD], np.float16).view(np.uint16).reshape(H, D))
        assert np.array_equal(vc[cache], np.asarray(qkv[2 * HD:], np.float16).view(np.uint16).reshape(H, D))
        O64, A, R = orc.attention_f64(q, kc, vc, 1, cache + 1, H, D, False, 1.0 / np.sqrt(D))
        got = io["o"][layer].download(np.float32, HD).astype(np.float64).reshape(1, H, D)
        tol = ((2.0 ** -10 + (cache + 1) * 2.0 ** -24 + 2 * D * 2.0 ** -24 * R[..., None]) * A
               + np.abs(O64) * 2.0 ** -24 + 1e-12)
        assert np.all(np.abs(got - O64) <= tol), layer
    logits = io["y"][-1].download(np.float32, 51200)
    want = orc.argmax(logits, m.F32, 1, 51200, 51200)[0]
    assert int(io["token"].download(np.int32, 1)[0]) == int(want)
    plan.destroy()
    for W in weights:
        W.free()
