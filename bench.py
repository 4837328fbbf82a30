#!/usr/bin/env python3
"""Benchmark of the MVLM matmul hot path on one MI355X.

Headline (one JSON line on stdout): decode GEMV HBM GB/s for one full Phi-1.5
decode step over Q8_0 weights -- 24 layers x {QKV 2048->6144, dense
2048->2048, fc1 2048->8192, fc2 8192->2048} + LM head 2048->51200, M = 1,
97 GEMVs, 1.3949 GB of GGUF-sized weights -- with inputs resident in HBM.
A step is one pass of the 97 GEMVs, enqueued from native code as a replayed
HIP graph.  The other configurations (Q4_0 at M = 1, 4, 16; the fp32 GEMV;
the M = 768 Phi-1.5 prefill GEMMs; the 729-token SigLIP GEMMs and the batched
Q*K^T; fused attention and the LM-head token pick) are reported under "extra"
with their own roofline fractions.

    python bench.py [--steps K] [--warmup W] [--quick] [--no-cpu] [--attention-only]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
import zlib

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0        # MI355X HBM3E, nominal
PEAK_F16_TFLOPS = 2500.0     # MI355X dense fp16/bf16 MFMA, nominal
SEED = 0x4D564C4D

PHI_LAYER = [("qkv", 6144, 2048), ("dense", 2048, 2048), ("fc1", 8192, 2048), ("fc2", 2048, 8192)]
PHI_LM_HEAD = ("lm_head", 51200, 2048)
PHI_STEP = [s for _ in range(24) for s in PHI_LAYER] + [PHI_LM_HEAD]


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def quant_bytes(qt, N, K):
    """GGUF bytes of a quantized [N,K] weight: 34 (Q8_0) or 18 (Q4_0) per 32 weights."""
    return N * (K // 32) * (34 if qt == "q8_0" else 18)


def gemv_bytes(qt, N, K, M):
    return quant_bytes(qt, N, K) + 4 * M * K + 4 * M * N


# Peaks derived from the device's own properties (mvlm_device_info box_peak_*),
# reported beside the nominal ones; set by main() once the device is open.
BOX_PEAK = {}


def roofline(bound, achieved, timing):
    """roofline block of one workload: achieved GB/s (bound "hbm") or TFLOP/s
    (bound "mfma") against MI355X's nominal peak, and against the peak derived
    from this device's reported clocks and CU count"""
    peak, unit = (PEAK_HBM_GBS, "GB/s") if bound == "hbm" else (PEAK_F16_TFLOPS, "TFLOP/s")
    r = {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
         "frac": round(achieved / peak, 4), "timing": timing}
    if BOX_PEAK.get(bound):
        r["peak_box"] = round(BOX_PEAK[bound], 1)
        r["frac_box"] = round(achieved / BOX_PEAK[bound], 4)
    return r


def timed_plan(dev, plan, steps, warmup):
    """Wall-clock device time of `steps` plan runs after `warmup` runs (ms per run)."""
    plan.run(warmup)
    dev.sync()
    t0 = dev.marker()
    plan.run(steps)
    t1 = dev.marker()
    dev.sync()
    import ctypes
    from mvlm_amd import native
    ms = ctypes.c_float()
    native.check(native.lib().mvlm_marker_elapsed_ms(t0.handle, t1.handle, ctypes.byref(ms)), "marker")
    return ms.value / steps


def profile_plan(plan, reps=5):
    """Per-launch kernel execution time: median over eager runs in which each launch
    carries HIP start/stop events on its own dispatch packet."""
    runs = np.stack([plan.profile() for _ in range(reps)])
    return np.median(runs, axis=0)


# ---------------------------------------------------------------------------
# workloads
# ---------------------------------------------------------------------------

def decode_inputs(dev, m, M):
    """The three activation inputs of a decode step: the block input (QKV, fc1 and
    the LM head read it), the attention output (dense) and the MLP hidden (fc2)."""
    ln = dev.fill_normal(dev.alloc(M * 2048 * 4), m.F32, M * 2048, SEED ^ 0x11, 1.0)
    attn = dev.fill_normal(dev.alloc(M * 2048 * 4), m.F32, M * 2048, SEED ^ 0x12, 1.0)
    gelu = dev.fill_normal(dev.alloc(M * 8192 * 4), m.F32, M * 8192, SEED ^ 0x13, 1.0)
    return {"qkv": ln, "fc1": ln, "dense": attn, "fc2": gelu, "lm_head": ln}


def build_decode_plan(dev, m, qt, M, grouped=True):
    """The plan of one Phi-1.5 decode step over quantized weights, M rows of
    activations (see decode_step); every GEMV writes its own output buffer and
    every stage reads the outputs of the stage before it, as in the model:
    QKV and fc1 of layer l+1 read fc2's output of layer l (layer 0: the block
    input), dense reads the first M x 2048 values of its layer's QKV output
    (the attention output's stand-in), fc2 reads fc1's output, and the LM head
    reads the last fc2 output.
    Returns (plan, weights, grouped, io) with io = {"x": input of each GEMV in
    PHI_STEP order, "y": outputs in PHI_STEP order}."""
    qdt = m.Q8_0 if qt == "q8_0" else m.Q4_0
    weights = [dev.random_weight(qdt, N, K, SEED ^ (0x100 + i), 0.02) for i, (_, N, K) in enumerate(PHI_STEP)]
    x_of = decode_inputs(dev, m, M)
    ys = [dev.alloc(M * N * 4) for _, N, _ in PHI_STEP]
    xs = []
    for layer in range(24):
        i0 = 4 * layer
        block_in = x_of["qkv"] if layer == 0 else ys[i0 - 1]
        xs += [block_in, ys[i0].view(0, M * 2048 * 4), block_in, ys[i0 + 2]]
    xs.append(ys[-2])
    plan = m.Plan(dev)
    if grouped:
        for layer in range(24):
            i0 = 4 * layer
            for pair in ((i0, i0 + 2), (i0 + 1, i0 + 3)):   # {QKV, fc1}, {dense, fc2}
                entries = [(xs[i], m.F32, weights[i], ys[i], m.F32) for i in pair]
                if M == 1:
                    plan.add_gemv_grouped(entries)
                else:
                    plan.add_gemm_quant_grouped(M, entries)
        plan.add_gemv(xs[-1], m.F32, weights[-1], ys[-1], m.F32, M)
    else:
        for x, W, y in zip(xs, weights, ys):
            plan.add_gemv(x, m.F32, W, y, m.F32, M)
    return plan, weights, grouped, {"x": xs, "y": ys, "inputs": x_of}


def decode_step(dev, m, qt, M, steps, warmup, graph=True, grouped=True):
    """One Phi-1.5 decode step over quantized weights, M rows of activations.

    Phi-1.5 blocks are parallel (attention and MLP read the same normalised
    input), so per layer QKV and fc1 are independent of each other, and so are
    dense (on the attention output) and fc2 (on the GELU output).  grouped=True
    issues each independent pair as one grouped launch (2 launches per layer +
    the LM head = 49); grouped=False issues the 97 GEMVs one launch each."""
    plan, weights, grouped, _ = build_decode_plan(dev, m, qt, M, grouped)
    per_op = profile_plan(plan)
    if graph:
        plan.use_graph(True)
    ms = timed_plan(dev, plan, steps, warmup)
    op_bytes = np.array([gemv_bytes(qt, N, K, M) for _, N, K in PHI_STEP], np.float64)
    step_bytes = float(op_bytes.sum())
    kernel_ms = float(per_op.sum())
    if grouped:
        launch_names = ["qkv+fc1", "dense+fc2"] * 24 + ["lm_head"]
    else:
        launch_names = [name for name, _, _ in PHI_STEP]
    res = {
        "workload": f"phi15_decode_{qt}_m{M}" + ("" if grouped else "_ungrouped"), "M": M,
        "gemvs": len(PHI_STEP), "launches": len(launch_names),
        "bytes_per_step": step_bytes, "ms_per_step": ms, "gbs": step_bytes / ms / 1e6,
        "kernel_ms_sum": kernel_ms, "kernel_gbs": step_bytes / kernel_ms / 1e6,
        "flops_per_step": float(sum(2.0 * M * N * K for _, N, K in PHI_STEP)),
        "per_launch_us": {name: float(np.median(per_op[[i for i, s in enumerate(launch_names) if s == name]]) * 1e3)
                          for name in dict.fromkeys(launch_names)},
    }
    res["frac"] = res["gbs"] / PEAK_HBM_GBS
    res["kernel_frac"] = res["kernel_gbs"] / PEAK_HBM_GBS
    res["roofline"] = roofline("hbm", res["gbs"], "timed region (HIP events around the graph replays) / launches")
    plan.destroy()
    for W in weights:
        W.free()
    return res


def build_token_plan(dev, m, qt, cache, fuse=True):
    """The plan of one Phi-1.5 decode step with the path's own ops end to end, in
    the reference's order (moondream2.cpp:359-541): per layer the grouped
    {QKV, fc1} GEMV; the decode attention step, which takes q and the new key
    and value from the QKV output, appends them (fp16) to the layer's KV cache
    at row `cache` and attends over cache + 1 keys (32 heads of 64, fp32
    output; kv_cache_append and attention_decode, moondream2.cpp:404-440); the
    grouped {dense, fc2} GEMV with dense reading the attention output; then the
    LM head and the on-device token pick.  Layer norm, the rotary embedding and
    the block's residual sum are not part of this path: every layer reads the
    same stand-in activations, and its cache holds `cache` random fp16 rows.
    The grouped launches carry the epilogues of the block's projections:
    QKV + bias, fc1 + bias + GELU, dense + bias + residual, fc2 + bias +
    residual (each branch writes its own output).  fuse: plan fusion, each
    attention step computed inside the {QKV, fc1} launch that writes its
    q, k and v (74 entries, 50 launches); off, every entry is a launch.
    Returns (plan, weights, io) with io = {"x" (input of each GEMV), "y"
    (PHI_STEP order), "ep" (per GEMV: dict of bias / act / residual buffers,
    or None), "token", "kc", "vc", "o" (per layer)}."""
    qdt = m.Q8_0 if qt == "q8_0" else m.Q4_0
    weights = [dev.random_weight(qdt, N, K, SEED ^ (0x100 + i), 0.02) for i, (_, N, K) in enumerate(PHI_STEP)]
    x_of = decode_inputs(dev, m, 1)
    ys = [dev.alloc(N * 4) for _, N, _ in PHI_STEP]
    h = dev.fill_normal(dev.alloc(2048 * 4), m.F32, 2048, SEED ^ 0x14, 1.0)        # residual stream
    bias = {name: dev.fill_normal(dev.alloc(N * 4), m.F32, N, SEED ^ (0x20 + j), 0.02)
            for j, (name, N, _) in enumerate(PHI_LAYER)}
    ep_of = {"qkv": {"bias": bias["qkv"]}, "fc1": {"bias": bias["fc1"], "act": m.native.ACT_GELU_TANH},
             "dense": {"bias": bias["dense"], "residual": h}, "fc2": {"bias": bias["fc2"], "residual": h}}
    eps = [ep_of.get(name) for name, _, _ in PHI_STEP]
    H, D = 32, 64
    rows = (cache + 1) * H * D
    kc = [dev.fill_normal(dev.alloc(rows * 2), m.F16, rows, SEED ^ (0x7000 + l), 1.0) for l in range(24)]
    vc = [dev.fill_normal(dev.alloc(rows * 2), m.F16, rows, SEED ^ (0x7100 + l), 1.0) for l in range(24)]
    o = [dev.alloc(H * D * 4) for _ in range(24)]
    tok = dev.alloc(4)
    plan = m.Plan(dev)
    plan.set_fusion(fuse)
    for layer in range(24):
        i0 = 4 * layer
        plan.add_gemv_grouped([(x_of["qkv"], m.F32, weights[i0], ys[i0], m.F32),
                               (x_of["fc1"], m.F32, weights[i0 + 2], ys[i0 + 2], m.F32)],
                              epilogues=[eps[i0], eps[i0 + 2]])
        plan.add_attention_decode_step(ys[i0], kc[layer], vc[layer], o[layer], cache, H, D)
        plan.add_gemv_grouped([(o[layer], m.F32, weights[i0 + 1], ys[i0 + 1], m.F32),
                               (x_of["fc2"], m.F32, weights[i0 + 3], ys[i0 + 3], m.F32)],
                              epilogues=[eps[i0 + 1], eps[i0 + 3]])
    plan.add_gemv(x_of["lm_head"], m.F32, weights[-1], ys[-1], m.F32, 1)
    plan.add_argmax(ys[-1], m.F32, 1, 51200, 51200, tok)
    xs = [v for layer in range(24) for v in (x_of["qkv"], o[layer], x_of["fc1"], x_of["fc2"])] + [x_of["lm_head"]]
    return plan, weights, {"x": xs, "y": ys, "ep": eps, "token": tok, "kc": kc, "vc": vc, "o": o}


def decode_token(dev, m, qt, cache, steps, warmup, fuse=True):
    """One Phi-1.5 decode step with the path's own ops end to end (build_token_plan)."""
    plan, weights, _ = build_token_plan(dev, m, qt, cache, fuse)
    fused = plan.fused()
    plan.use_graph(True)
    ms = timed_plan(dev, plan, steps, warmup)
    plan.check()
    plan.destroy()
    for W in weights:
        W.free()
    nbytes = (sum(gemv_bytes(qt, N, K, 1) for _, N, K in PHI_STEP)   # weights, x, y
              + 24 * 2 * (cache + 1) * 32 * 64 * 2.0                  # each layer's KV cache, fp16 (+ the append)
              + 51200 * 4.0)                                          # logits read by the token pick
    kernels = 24 * 2 + 2 + (0 if fused else 24 * (2 if cache > 128 else 1))   # an unfused step: split + merge
    return {"workload": f"phi15_decode_token_{qt}_cache{cache}" + ("" if fuse else "_unfused"), "us": ms * 1e3,
            "tokens_per_s": 1e3 / ms, "ops": 24 * 3 + 2, "kernels": kernels,
            "attention": ("each layer's attention step (cache append + attention over cache + 1 keys) computed "
                          "inside the {QKV, fc1} launch that writes its q, k, v (plan fusion)" if fused
                          else "one attention step launch per layer (split kernel + merge kernel)"),
            "epilogues": "QKV+bias, fc1+bias+GELU, dense+bias+residual, fc2+bias+residual "
                         "fused into the grouped GEMVs",
            "bytes_per_token": nbytes,
            "roofline": roofline("hbm", nbytes / ms / 1e6, "timed region (HIP events around the graph replays) "
                                 "/ tokens; bytes = weights, x and y of the 97 GEMVs, the KV cache, the logits")}


def token_extras(dev, m, steps, warmup, extra):
    for qt, cache, fuse in (("q8_0", 512, True), ("q8_0", 512, False), ("q8_0", 2048, True), ("q4_0", 512, True)):
        r = decode_token(dev, m, qt, cache, steps, warmup, fuse)
        extra[r["workload"]] = r
        log(f"[bench]   {r['workload']}: {r['us']:.1f} us/token ({r['tokens_per_s']:.0f} tokens/s; GEMVs, "
            f"attention, LM head and token pick, one graph of {r['kernels']} kernel launches)")


def fp32_gemv(dev, m, steps, warmup, copies=16):
    """x[1x2048] . W[2048x8192] fp32 (gemm_bench.cpp's llm_ffn shape), rotating over
    `copies` weight copies (16 x 67 MB > the 256 MB Infinity Cache)."""
    N, K = 8192, 2048
    weights = [dev.random_weight(m.F32, N, K, SEED ^ (0x200 + i), 0.02) for i in range(copies)]
    x = dev.fill_normal(dev.alloc(K * 4), m.F32, K, SEED ^ 0x201, 1.0)
    y = dev.alloc(N * 4)
    plan = m.Plan(dev)
    for W in weights:
        plan.add_gemv(x, m.F32, W, y, m.F32)
    per_op = profile_plan(plan)
    plan.use_graph(True)
    ms = timed_plan(dev, plan, steps, warmup) / copies
    nbytes = 4.0 * N * K + 4 * K + 4 * N
    res = {"workload": "gemv_f32_2048x8192", "us": ms * 1e3, "gbs": nbytes / ms / 1e6,
           "kernel_us": float(np.median(per_op)) * 1e3, "kernel_gbs": nbytes / float(np.median(per_op)) / 1e6}
    res["frac"] = res["gbs"] / PEAK_HBM_GBS
    res["roofline"] = roofline("hbm", res["gbs"], "timed region (HIP events around the graph replays of "
                               f"{copies} launches, one per weight copy) / launches")
    plan.destroy()
    return res


def gemv_exact(dev, m, steps, warmup, copies=16):
    """mvlm_gemv_exact (the reference gemv's summation order, fp16 in and out) at
    x[1x2048] . W[2048x8192], rotating over `copies` 32 MB packed fp16 weights."""
    N, K = 8192, 2048
    Bs = [dev.random_weight(m.F16, N, K, SEED ^ (0x300 + i), 0.02) for i in range(copies)]
    x = dev.fill_normal(dev.alloc(K * 2), m.F16, K, SEED ^ 0x301, 1.0)
    y = dev.alloc(N * 2)
    for i in range(warmup):
        dev.gemv_exact(x, Bs[i % copies], y, N, K)
    dev.sync()
    times = []
    for i in range(max(steps, copies)):
        ev = dev.gemv_exact(x, Bs[i % copies], y, N, K, event=True)
        ev.wait()
        times.append(ev.elapsed_ms())
    us = float(np.median(times)) * 1e3
    nbytes = 2.0 * N * K + 2 * K + 2 * N
    return {"workload": "gemv_exact_f16_2048x8192", "kernel_us": us, "gbs": nbytes / us / 1e3,
            "frac": nbytes / us / 1e3 / PEAK_HBM_GBS,
            "roofline": roofline("hbm", nbytes / us / 1e3, "median of per-launch HIP start/stop events, "
                                 f"rotating over {copies} weight copies")}


def gemm_shape(dev, m, name, M, N, K, steps, warmup, bf16=False):
    """fp16-in (bf16 with bf16=True) / fp32-out MFMA GEMM, A[M,K] N(0,1), W[N,K] N(0,0.02)."""
    dt = m.BF16 if bf16 else m.F16
    W = dev.random_weight(dt, N, K, SEED ^ (zlib.crc32(name.encode()) & 0xFFFF), 0.02)
    A = dev.fill_normal(dev.alloc(M * K * 2), dt, M * K, SEED ^ 0x300, 1.0)
    C = dev.alloc(M * N * 4)
    plan = m.Plan(dev)
    plan.add_gemm_packed(A, dt, W, C, m.F32, M)
    per_op = profile_plan(plan)
    ms = timed_plan(dev, plan, steps, warmup)
    flops = 2.0 * M * N * K
    res = {"workload": name, "shape": [M, N, K], "dtype": "bf16" if bf16 else "f16", "us": ms * 1e3,
           "tflops": flops / ms / 1e9, "kernel_us": float(per_op[0]) * 1e3}
    res["frac"] = res["tflops"] / PEAK_F16_TFLOPS
    res["roofline"] = roofline("mfma", res["tflops"], "timed region (HIP events around the graph replays) / launches")
    plan.destroy()
    return res


def qk_batched(dev, m, steps, warmup):
    H, S, D = 16, 729, 72
    Q = dev.fill_normal(dev.alloc(S * H * D * 2), m.F16, S * H * D, SEED ^ 0x401, 1.0)
    Kt = dev.fill_normal(dev.alloc(S * H * D * 2), m.F16, S * H * D, SEED ^ 0x402, 1.0)
    C = dev.alloc(H * S * S * 4)
    plan = m.Plan(dev)
    plan.add_gemm_batched(Q, Kt, C, H, S, S, D, H * D, H * D, S, D, D, S * S)
    ms = timed_plan(dev, plan, steps, warmup)
    flops = 2.0 * H * S * S * D
    nbytes = 2.0 * 2 * S * H * D + 4.0 * H * S * S
    res = {"workload": "siglip_qk_16x729x729x72", "us": ms * 1e3, "tflops": flops / ms / 1e9,
           "gbs": nbytes / ms / 1e6}
    res["frac_mfma"] = res["tflops"] / PEAK_F16_TFLOPS
    res["frac_hbm"] = res["gbs"] / PEAK_HBM_GBS
    timing = "timed region (HIP events around the graph replays) / launches"
    res["roofline"] = roofline("hbm", res["gbs"], timing + "; bytes = fp16 Q and K + fp32 scores")
    res["roofline_mfma"] = roofline("mfma", res["tflops"], timing)
    plan.destroy()
    return res


ATTENTION_SHAPES = [
    # name, seq_q, seq_kv, heads, head_dim, causal
    ("siglip_attention_16x729x72", 729, 729, 16, 72, False),
    ("phi15_prefill_attention_768_causal", 768, 768, 32, 64, True),
    ("phi15_decode_attention_cache2048", 1, 2048, 32, 64, False),
    ("phi15_decode_attention_cache512", 1, 512, 32, 64, False),
]


# Short single ops are timed as OP_REPEATS back-to-back copies in one plan
# (one graph replay), so the per-op time is not one graph launch's host cost.
OP_REPEATS = 16


def attention_shape(dev, m, name, sq, skv, H, D, causal, steps, warmup):
    """Fused attention, fp16 Q/K/V ~ N(0,1) in [seq][heads][head_dim], fp16 out.
    flops = 4 H sq skv D (QK^T and PV; half of it under a square causal mask);
    bytes = Q + K + V + O once each.  `us`: per op within a graph of OP_REPEATS
    copies; `kernel_us`: median device time of one copy (HIP events)."""
    n = sq * H * D
    Q = dev.fill_normal(dev.alloc(n * 2), m.F16, n, SEED ^ 0x501, 1.0)
    K = dev.fill_normal(dev.alloc(skv * H * D * 2), m.F16, skv * H * D, SEED ^ 0x502, 1.0)
    V = dev.fill_normal(dev.alloc(skv * H * D * 2), m.F16, skv * H * D, SEED ^ 0x503, 1.0)
    O = dev.alloc(n * 2)
    plan = m.Plan(dev)
    for _ in range(OP_REPEATS):
        plan.add_attention(Q, K, V, O, m.F16, sq, skv, H, D, causal=causal)
    per_op = profile_plan(plan)
    plan.use_graph(True)
    ms = timed_plan(dev, plan, steps, warmup) / OP_REPEATS
    frac_causal = (1.0 - (sq - 1) / (2.0 * skv)) if causal else 1.0
    flops = 4.0 * H * sq * skv * D * frac_causal
    nbytes = 2.0 * (2 * sq * H * D + 2 * skv * H * D)
    kus = float(np.median(per_op)) * 1e3
    res = {"workload": name, "shape": [sq, skv, H, D, int(causal)], "us": ms * 1e3, "kernel_us": kus,
           "tflops": flops / kus / 1e6, "gbs": nbytes / kus / 1e3}
    res["frac_mfma"] = res["tflops"] / PEAK_F16_TFLOPS
    res["frac_hbm"] = res["gbs"] / PEAK_HBM_GBS
    timing = "median of per-launch HIP start/stop events over one eager pass of the graph's copies"
    if sq == 1:   # one query: streaming the KV cache
        res["roofline"] = roofline("hbm", res["gbs"], timing + "; bytes = Q, K, V and O once each")
    else:
        res["roofline"] = roofline("mfma", res["tflops"], timing + "; flops = QK^T and PV (causal: visible half)")
    plan.destroy()
    return res


def token_pick(dev, m, steps, warmup):
    """Row argmax of 51200 fp32 logits (the LM-head token pick)."""
    n = PHI_LM_HEAD[1]
    x = dev.fill_normal(dev.alloc(n * 4), m.F32, n, SEED ^ 0x601, 1.0)
    out = dev.alloc(4)
    plan = m.Plan(dev)
    for _ in range(OP_REPEATS):
        plan.add_argmax(x, m.F32, 1, n, n, out)
    per_op = profile_plan(plan)
    plan.use_graph(True)
    ms = timed_plan(dev, plan, steps, warmup) / OP_REPEATS
    kus = float(np.median(per_op)) * 1e3
    res = {"workload": "token_pick_51200_f32", "us": ms * 1e3, "kernel_us": kus, "gbs": 4.0 * n / kus / 1e3}
    res["roofline"] = roofline("hbm", res["gbs"], "median of per-launch HIP start/stop events; bytes = the "
                               "fp32 logits read once")
    plan.destroy()
    return res


# benchmarks/gemm_bench.cpp:16-22: name, M, K, N
GEMM_BENCH_CONFIGS = (("small", 256, 256, 256), ("medium", 2048, 2048, 2048), ("decode_gemv", 1, 2048, 2048),
                      ("llm_ffn", 1, 2048, 8192), ("prefill_32", 32, 2048, 2048))
GEMM_BENCH_VARIANTS = ("naive", "tiled", "image", "gemv", "gemv_exact")


def gemm_bench_matrix(dev, m, warmup=5, iters=20):
    """The reference bench's variant x config table (gemm_bench.cpp:16-22, 58-63,
    141-186): fp16 A[M,K] and B[K,N] (the reference's row-major B), fp16 C;
    naive / tiled (the reference kernels' exact fma order), image (the MFMA
    GEMM on B packed from the reference's [K,N] layout), gemv and gemv_exact
    (M = 1 only).  5 warmup launches, then 20 launches each timed by its own
    start/stop events; GFLOP/s = 2MKN / average time (gemm_bench.cpp:48-51),
    efficiency against the 2.5 PFLOP/s dense fp16 peak; GEMV rows also give
    GB/s over the fp16 weight + x + y bytes.  The same matrices are reused
    launch after launch, as in the reference bench, so they sit in the
    256 MB Infinity Cache."""
    rows = []
    for cname, M, K, N in GEMM_BENCH_CONFIGS:
        A = dev.fill_normal(dev.alloc(M * K * 2), m.F16, M * K, SEED ^ 0x801, 1.0)
        B = dev.fill_normal(dev.alloc(K * N * 2), m.F16, K * N, SEED ^ 0x802, 0.02)
        C = dev.alloc(M * N * 2)
        W = dev.pack(B.download(np.uint16, K * N), m.F16, N, K, layout=m.LAYOUT_KN)
        launch = {"naive": lambda ev: dev.gemm_naive(A, B, C, M, N, K, event=ev),
                  "tiled": lambda ev: dev.gemm_tiled(A, B, C, M, N, K, event=ev),
                  "image": lambda ev: dev.gemm_packed(A, m.F16, W, C, m.F16, M, N, K, event=ev),
                  "gemv": lambda ev: dev.gemv(A, m.F16, W, C, m.F16, N, K, event=ev),
                  "gemv_exact": lambda ev: dev.gemv_exact(A, W, C, N, K, event=ev)}
        for v in GEMM_BENCH_VARIANTS:
            if v.startswith("gemv") and M != 1:
                continue
            run = launch[v]
            for _ in range(warmup):
                run(False)
            dev.sync()
            ts = []
            for _ in range(iters):
                ev = run(True)
                ev.wait()
                ts.append(ev.elapsed_ms())
            avg = float(np.mean(ts))
            gf = 2.0 * M * K * N / (avg * 1e6)
            r = {"variant": v, "config": cname, "M": M, "K": K, "N": N, "avg_ms": avg, "min_ms": float(min(ts)),
                 "max_ms": float(max(ts)), "gflops": gf, "eff_pct_of_2.5PF": 100.0 * gf / (PEAK_F16_TFLOPS * 1e3)}
            if M == 1:
                r["gbs"] = (2.0 * K * N + 2 * K + 2 * N) / (avg * 1e6)
            rows.append(r)
            log(f"[bench]   {v:10s} {cname:12s} {M:4d}x{K:4d}x{N:4d} {avg:8.4f} ms {gf:10.1f} GFLOPS "
                f"{r['eff_pct_of_2.5PF']:5.2f}% eff" + (f" {r['gbs']:7.0f} GB/s" if M == 1 else ""))
        W.free()
    return rows


GEMM_SHAPES = (("phi15_prefill_qkv", 768, 6144, 2048), ("phi15_prefill_fc1", 768, 8192, 2048),
               ("phi15_prefill_fc2", 768, 2048, 8192), ("siglip_qkv", 729, 3456, 1152),
               ("siglip_out", 729, 1152, 1152), ("siglip_fc1", 729, 4304, 1152),
               ("siglip_fc2", 729, 1152, 4304))


def gemm_extras(dev, m, steps, warmup, extra):
    """The M = 729 / 768 fp16 GEMMs (Phi-1.5 prefill, SigLIP) and the batched QK^T."""
    for bf16 in (False, True):
        for name, M, N, K in GEMM_SHAPES:
            r = gemm_shape(dev, m, name + ("_bf16" if bf16 else ""), M, N, K, steps, warmup, bf16)
            extra[r["workload"]] = r
            log(f"[bench]   {r['workload']} {M}x{N}x{K}: {r['us']:.1f} us {r['tflops']:.0f} TFLOP/s "
                f"({100 * r['frac']:.1f}% of 2.5 PF)")
    r = qk_batched(dev, m, steps, warmup)
    extra[r["workload"]] = r
    log(f"[bench]   {r['workload']}: {r['us']:.1f} us {r['tflops']:.0f} TFLOP/s {r['gbs']:.0f} GB/s")


def f4_extras(dev, m, steps, warmup, extra):
    for name, sq, skv, H, D, causal in ATTENTION_SHAPES:
        r = attention_shape(dev, m, name, sq, skv, H, D, causal, steps, warmup)
        extra[name] = r
        log(f"[bench]   {name}: {r['kernel_us']:.1f} us kernel ({r['us']:.1f} us per op in a graph of {OP_REPEATS}) "
            f"{r['tflops']:.0f} TFLOP/s ({100 * r['frac_mfma']:.1f}% of 2.5 PF) {r['gbs']:.0f} GB/s")
    r = token_pick(dev, m, steps, warmup)
    extra[r["workload"]] = r
    log(f"[bench]   {r['workload']}: {r['kernel_us']:.1f} us kernel ({r['us']:.1f} us per op in a graph of {OP_REPEATS})")


# ---------------------------------------------------------------------------
# CPU baseline: the oracle's Q8_0 GEMV on the host cores
# ---------------------------------------------------------------------------

def cpu_baseline(seconds=10.0):
    from oracle import oracle_ffi as orc
    threads = orc.lib().orc_max_threads()
    x2, x8 = orc.normal_f32(2048, SEED ^ 1), orc.normal_f32(8192, SEED ^ 2)
    layer = [(orc.q8_0_blocks(N * K // 32, SEED ^ (0x500 + i)), N, K) for i, (_, N, K) in enumerate(PHI_LAYER)]
    nbytes = sum(gemv_bytes("q8_0", N, K, 1) for _, N, K in layer)
    for W, N, K in layer:    # warm-up
        orc.gemm_nk("q8_0", x2 if K == 2048 else x8, W, 1, N, K, threads)
    reps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for W, N, K in layer:
            orc.gemm_nk("q8_0", x2 if K == 2048 else x8, W, 1, N, K, threads)
        reps += 1
    dt = time.perf_counter() - t0
    # the same sample on one thread, for a third of the time
    reps1, t1 = 0, time.perf_counter()
    while time.perf_counter() - t1 < seconds / 3:
        for W, N, K in layer:
            orc.gemm_nk("q8_0", x2 if K == 2048 else x8, W, 1, N, K, 1)
        reps1 += 1
    dt1 = time.perf_counter() - t1
    return {"value": nbytes * reps / dt / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{reps} passes over one Phi-1.5 layer's 4 Q8_0 GEMVs (QKV, dense, fc1, fc2; "
                      f"{nbytes / 1e6:.1f} MB each pass) in {dt:.1f} s: dequantize each 32-block exactly, "
                      f"fp32 fma over ascending k, OpenMP over rows",
            "single_thread_value": nbytes * reps1 / dt1 / 1e9,
            "single_thread_sample": f"{reps1} passes of the same layer on 1 thread in {dt1:.1f} s",
            "legs": cpu_reference_legs(threads)}


def _timed(fn, seconds):
    """calls fn until `seconds` have passed (at least twice, the first untimed); returns (calls, s)"""
    fn()
    n, t0 = 0, time.perf_counter()
    while n < 1 or time.perf_counter() - t0 < seconds:
        fn()
        n += 1
    return n, time.perf_counter() - t0


def cpu_reference_legs(threads, seconds=1.5):
    """The oracle's restatements of the reference kernels themselves, timed on the
    host in the units of their GPU rows: gemv (gemm.cl:219-270, fp16 x and W, the
    256-item partition and fold) at the fp32 GEMV's shape 1x2048x8192; the fp32
    NT GEMV (C1: x[2048] fp32, W[8192][2048] fp32, ascending-k fma); gemm_image
    (gemm.cl:157-200) on a slice of 4 rows per thread of the Phi-1.5 QKV prefill
    GEMM (768x6144x2048: each row is an independent work item, so the rate
    carries over).  Each on all `threads` and on one thread."""
    from oracle import oracle_ffi as orc
    legs = []
    K, N = 2048, 8192
    x16, B16 = orc.normal_f16(K, SEED ^ 0x901), orc.normal_f16(K * N, SEED ^ 0x902, 0.02)
    x32, W32 = orc.normal_f32(K, SEED ^ 0x903), orc.normal_f32(N * K, SEED ^ 0x904, 0.02)
    Nq, Kq = 6144, 2048
    Aq, Bq = orc.normal_f16(4 * threads * Kq, SEED ^ 0x905), orc.normal_f16(Kq * Nq, SEED ^ 0x906, 0.02)
    for nt in (threads, 1):
        Mq = 4 * nt
        n, dt = _timed(lambda: orc.gemv(x16, B16, N, K, nthreads=nt), seconds)
        legs.append({"kernel": "gemv (gemm.cl:219-270)", "shape": "1x2048x8192 fp16", "threads": nt,
                     "gbs": (2.0 * K * N + 2 * K + 2 * N) * n / dt / 1e9, "us": dt / n * 1e6})
        n, dt = _timed(lambda: orc.gemm_nk("f32", x32, W32, 1, N, K, nt), seconds)
        legs.append({"kernel": "fp32 NT GEMV (C1)", "shape": "1x2048x8192 fp32", "threads": nt,
                     "gbs": (4.0 * K * N + 4 * K + 4 * N) * n / dt / 1e9, "us": dt / n * 1e6})
        n, dt = _timed(lambda: orc.gemm_image_mt(Aq, Bq, Mq, Nq, Kq, nt), seconds)
        legs.append({"kernel": "gemm_image (gemm.cl:157-200)", "shape": f"{Mq}x6144x2048 slice of 768x6144x2048 fp16",
                     "threads": nt, "gflops": 2.0 * Mq * Nq * Kq * n / dt / 1e9, "ms": dt / n * 1e3})
    return legs


# ---------------------------------------------------------------------------
# HBM traffic of the headline step from rocprofv3 counters
# ---------------------------------------------------------------------------

TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_phi15_decode_q8_0.json")
COPY_BYTES = 256 << 20


def pmc_probe(steps=3):
    """Workload for the counter runs: `steps` eager headline steps (49 kernels
    each), then a plain device-to-device copy of COPY_BYTES (the calibration:
    what FETCH_SIZE / WRITE_SIZE read for a kernel of known traffic)."""
    import mvlm_amd as m
    import torch
    dev = m.Device(0)
    plan, weights, _, _ = build_decode_plan(dev, m, "q8_0", 1, True)
    plan.run(1)
    dev.sync()
    plan.run(steps)
    dev.sync()
    src = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    plan.destroy()
    for W in weights:
        W.free()
    dev.close()
    print("pmc probe done", flush=True)


PMC_WORKLOADS = ("decode_q8_0_m1", "decode_q4_0_m1", "decode_q4_0_m4", "decode_q4_0_m16", "decode_q8_0_m4", "gemm",
                 "gemm_bf16", "gemm_vendor", "gemv_f32", "gemv_exact", "qk_batched", "attention", "argmax", "token")


def pmc_workload(name, reps=2):
    """Workload of a counter run (rocprofv3 --pmc): `reps` eager passes of one
    decode step (decode_<qt>_m<M>, grouped like the bench) or of every GEMM
    shape of --gemm-only (one launch plan each), then the calibration copy of
    pmc_probe.  Prints one line per pass."""
    import mvlm_amd as m
    import torch
    dev = m.Device(0)
    plans, weights = [], []
    if name.startswith("decode_"):
        _, qt0, qt1, mm = name.split("_")
        plan, ws, _, _ = build_decode_plan(dev, m, f"{qt0}_{qt1}", int(mm[1:]), True)
        plans.append((name, plan))
        weights += ws
    elif name in ("gemm", "gemm_bf16"):
        dt = m.BF16 if name == "gemm_bf16" else m.F16
        for wname, M, N, K in GEMM_SHAPES:
            W = dev.random_weight(dt, N, K, SEED ^ (zlib.crc32(wname.encode()) & 0xFFFF), 0.02)
            A = dev.fill_normal(dev.alloc(M * K * 2), dt, M * K, SEED ^ 0x300, 1.0)
            C = dev.alloc(M * N * 4)
            plan = m.Plan(dev)
            plan.add_gemm_packed(A, dt, W, C, m.F32, M)
            plans.append((wname, plan))
            weights.append(W)
    elif name in ("gemv_f32", "gemv_exact"):   # 16 rotating copies of the 2048 -> 8192 weight
        N, K = 8192, 2048
        dt = m.F32 if name == "gemv_f32" else m.F16
        x = dev.fill_normal(dev.alloc(K * 4), dt, K, SEED ^ 0x201, 1.0)
        y = dev.alloc(N * 4)
        plan = m.Plan(dev)
        for i in range(16):
            W = dev.random_weight(dt, N, K, SEED ^ (0x200 + i), 0.02)
            weights.append(W)
            if name == "gemv_f32":
                plan.add_gemv(x, m.F32, W, y, m.F32)
        if name == "gemv_exact":
            class Exact:   # one eager pass: each copy through mvlm_gemv_exact
                def run(self, n):
                    for W in weights:
                        dev.gemv_exact(x, W, y, N, K)

                def destroy(self):
                    pass
            plan.destroy()
            plan = Exact()
        plans.append((name, plan))
    elif name == "qk_batched":
        H, S, D = 16, 729, 72
        Q = dev.fill_normal(dev.alloc(S * H * D * 2), m.F16, S * H * D, SEED ^ 0x401, 1.0)
        Kt = dev.fill_normal(dev.alloc(S * H * D * 2), m.F16, S * H * D, SEED ^ 0x402, 1.0)
        C = dev.alloc(H * S * S * 4)
        plan = m.Plan(dev)
        plan.add_gemm_batched(Q, Kt, C, H, S, S, D, H * D, H * D, S, D, D, S * S)
        plans.append((name, plan))
    elif name == "attention":
        for aname, sq, skv, H, D, causal in ATTENTION_SHAPES:
            Q = dev.fill_normal(dev.alloc(sq * H * D * 2), m.F16, sq * H * D, SEED ^ 0x501, 1.0)
            K = dev.fill_normal(dev.alloc(skv * H * D * 2), m.F16, skv * H * D, SEED ^ 0x502, 1.0)
            V = dev.fill_normal(dev.alloc(skv * H * D * 2), m.F16, skv * H * D, SEED ^ 0x503, 1.0)
            O = dev.alloc(sq * H * D * 2)
            plan = m.Plan(dev)
            plan.add_attention(Q, K, V, O, m.F16, sq, skv, H, D, causal=causal)
            plans.append((aname, plan))
    elif name == "token":   # the Q8_0 token plan at cache 512, attention fused into the launches
        plan, ws, _ = build_token_plan(dev, m, "q8_0", 512, True)
        plans.append((name, plan))
        weights += ws
    elif name == "gemm_vendor":   # torch.matmul (the vendor library) on the Phi-1.5 QKV and fc1 shapes
        class Vendor:
            def __init__(self, M, N, K):
                g = torch.Generator(device="cuda").manual_seed(SEED)
                self.A = torch.randn(M, K, device="cuda", dtype=torch.float16, generator=g)
                self.W = torch.randn(N, K, device="cuda", dtype=torch.float16, generator=g) * 0.02

            def run(self, n):
                for _ in range(n):
                    torch.matmul(self.A, self.W.t())
                torch.cuda.synchronize()

            def destroy(self):
                pass
        for wname, M, N, K in GEMM_SHAPES[:2]:
            plans.append((wname, Vendor(M, N, K)))
    elif name == "argmax":
        n = PHI_LM_HEAD[1]
        x = dev.fill_normal(dev.alloc(n * 4), m.F32, n, SEED ^ 0x601, 1.0)
        out = dev.alloc(4)
        plan = m.Plan(dev)
        plan.add_argmax(x, m.F32, 1, n, n, out)
        plans.append((name, plan))
    else:
        raise SystemExit(f"unknown counter workload {name}; one of {', '.join(PMC_WORKLOADS)}")
    for r in range(reps):
        for pname, plan in plans:
            plan.run(1)
            dev.sync()
        print(f"pmc {name} pass {r} done", flush=True)
    src = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    for _, plan in plans:
        plan.destroy()
    for W in weights:
        W.free()
    dev.close()
    print("pmc probe done", flush=True)


def counter_table(dirs, kernel_filter=""):
    """Per (kernel, grid) mean per dispatch of every counter found in the
    counter_collection.csv files under `dirs`, as a markdown table (stdout)."""
    import csv
    import glob
    per = {}
    for d in dirs:
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            seen = {}
            for r in csv.DictReader(open(f)):
                name = r["Kernel_Name"]
                if kernel_filter not in name:
                    continue
                key = (name, r.get("Grid_Size", ""))
                disp = (f, int(r["Dispatch_Id"]))
                e = per.setdefault(key, {})
                c = e.setdefault(r["Counter_Name"], {})
                c[disp] = c.get(disp, 0.0) + float(r["Counter_Value"])
                seen[disp] = 1
    counters = sorted({c for e in per.values() for c in e})
    print("| kernel | grid | dispatches | " + " | ".join(counters) + " |")
    print("|---|---|---|" + "---|" * len(counters))
    for (name, grid), e in sorted(per.items()):
        n = max(len(v) for v in e.values())
        cells = [f"{np.mean(list(e[c].values())):.4g}" if c in e else "" for c in counters]
        short = name.split("(")[0].replace("void ", "")[:70]
        print(f"| `{short}` | {grid} | {n} | " + " | ".join(cells) + " |")


def _counter_rows(d):
    import csv
    import glob
    f = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
    if not f:
        raise SystemExit(f"no counter_collection.csv under {d}")
    per = {}
    for r in csv.DictReader(open(f[0])):
        key = int(r["Dispatch_Id"])
        e = per.setdefault(key, {"name": r["Kernel_Name"], "grid": int(r.get("Grid_Size", 0) or 0), "value": 0.0})
        e["value"] += float(r["Counter_Value"])
    return [per[k] for k in sorted(per)]


def pmc_summarize(fetch_dir, write_dir, out=TRAFFIC_FILE):
    """FETCH_SIZE / WRITE_SIZE (KiB per dispatch) of the last headline step and
    of the calibration copy -> HBM bytes per step, scaled by the copy's
    measured/true ratio."""
    res = {}
    for counter, d in (("fetch", fetch_dir), ("write", write_dir)):
        rows = _counter_rows(d)
        gemv = [r for r in rows if "gemv_stream_kernel" in r["name"]]
        copy = [r for r in rows if "copy" in r["name"].lower() or "elementwise" in r["name"].lower()]
        step = gemv[-49:]
        raw = sum(r["value"] for r in step) * 1024.0
        cal = (min(r["value"] for r in copy[-3:]) * 1024.0) / COPY_BYTES if copy else 1.0
        res[counter] = {"raw_bytes_per_step": raw, "copy_factor": cal, "bytes_per_step": raw / cal,
                        "copy_kernel": copy[-1]["name"][:80] if copy else None, "launches": len(step)}
    alg = float(sum(gemv_bytes("q8_0", N, K, 1) for _, N, K in PHI_STEP))
    total = res["fetch"]["bytes_per_step"] + res["write"]["bytes_per_step"]
    summary = {"workload": "phi15_decode_q8_0", "algorithmic_bytes_per_step": alg,
               "hbm_bytes_per_step": total, "ratio_to_algorithmic": total / alg, "fetch": res["fetch"],
               "write": res["write"],
               "command": "cd /tmp && export TMPDIR=/tmp && rocprofv3 --pmc FETCH_SIZE -d $OUT/pmc_fetch "
                          "-o run --output-format csv -- python3 $R/bench.py --pmc-workload decode_q8_0_m1; same "
                          "with WRITE_SIZE into $OUT/pmc_write; python3 $R/bench.py --pmc-summarize "
                          "$OUT/pmc_fetch $OUT/pmc_write   (R = repository root, OUT = an output directory; "
                          "--pmc-probe in place of --pmc-workload decode_q8_0_m1 gives the same step)"}
    with open(out, "w") as fh:
        json.dump(summary, fh, indent=1)
    print(json.dumps(summary, indent=1))


def measured_traffic():
    try:
        with open(TRAFFIC_FILE) as fh:
            return float(json.load(fh)["hbm_bytes_per_step"])
    except (OSError, ValueError, KeyError):
        return None


# ---------------------------------------------------------------------------

def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--quick", action="store_true", help="headline only, no extra workloads")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--eager", action="store_true", help="enqueue plans eagerly instead of replaying HIP graphs")
    ap.add_argument("--pmc-probe", action="store_true", help="workload for rocprofv3 --pmc traffic runs")
    ap.add_argument("--pmc-workload", choices=PMC_WORKLOADS,
                    help="workload for rocprofv3 --pmc counter runs (eager passes, see pmc_workload)")
    ap.add_argument("--counter-table", nargs="+", metavar="DIR",
                    help="markdown table of the counters collected under DIR(s) (per kernel and grid)")
    ap.add_argument("--kernel-filter", default="", help="with --counter-table: kernels whose name contains this")
    ap.add_argument("--attention-only", action="store_true",
                    help="only the attention and token-pick workloads (one JSON line of them)")
    ap.add_argument("--token-only", action="store_true",
                    help="only the decode-token plans (Q8_0 cache 512 fused and not, 2048; Q4_0 512; one JSON line)")
    ap.add_argument("--gemm-only", action="store_true",
                    help="only the prefill / vision GEMM shapes and the batched QK^T (one JSON line of them)")
    ap.add_argument("--gemm-bench", action="store_true",
                    help="only the reference bench's variant x config table (one JSON line)")
    ap.add_argument("--latency-probe", action="store_true",
                    help="first-load latency at kernel start (mvlm_probe_load_latency; one JSON line)")
    ap.add_argument("--barrier-probe", action="store_true",
                    help="software grid-barrier latency per round, each protocol with HBM idle and busy "
                         "(mvlm_probe_grid_barrier; one JSON line)")
    ap.add_argument("--pmc-summarize", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="turn the two counter runs into " + os.path.relpath(TRAFFIC_FILE, ROOT))
    args = ap.parse_args()
    if args.pmc_summarize:
        pmc_summarize(*args.pmc_summarize)
        return
    if args.pmc_probe:
        pmc_probe()
        return
    if args.pmc_workload:
        pmc_workload(args.pmc_workload)
        return
    if args.counter_table:
        counter_table(args.counter_table, args.kernel_filter)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this library has no multi-GPU path (the decode GEMV would shard "
              "along N, each GPU streaming its rows); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import mvlm_amd as m
    dev = m.Device(0)
    info = dev.info()
    BOX_PEAK["hbm"], BOX_PEAK["mfma"] = info.box_peak_hbm_gbs, info.box_peak_fp16_tflops
    log(f"[bench] {info.device_name.decode()} {info.arch_name.decode()} CUs={info.compute_units} "
        f"clock={info.max_clock_mhz} MHz HBM={info.global_mem_size / 2**30:.0f} GiB; derived peaks "
        f"{info.box_peak_fp16_tflops:.0f} TFLOP/s fp16 (CUs x clock x 4096), {info.box_peak_hbm_gbs:.0f} GB/s "
        f"(memory clock {info.memory_clock_mhz} MHz x {info.memory_bus_width_bits} bits x 4 / 8)")
    if args.barrier_probe:
        names = ["counter_atomic_poll", "flag_per_workgroup", "counter_replicated_done"]
        res = {}
        for bg in (False, True):
            for v, name in enumerate(names):
                key = f"{name}_{'hbm_busy' if bg else 'hbm_idle'}_us"
                runs = []
                for _ in range(3):
                    try:
                        runs.append(dev.probe_grid_barrier(v, 200, bg))
                    except m.native.MvlmError:   # a round waited more than 20 ms
                        runs.append(float("inf"))
                us = min(runs)
                res[key] = round(us, 2) if us != float("inf") else "gave up (a round > 20 ms)"
                log(f"[bench]   grid barrier {name:24s} HBM {'busy' if bg else 'idle'}: {res[key]} us/round")
        print(json.dumps({"grid_barrier_us_per_round": res}), flush=True)
        dev.close()
        return
    if args.latency_probe:
        res = {}
        for variant, vname in ((0, "from_hbm"), (1, "out_of_range")):
            for after in (0, 4, 9):
                runs = [dev.probe_load_latency(variant, after) for _ in range(3)]
                best = min(runs, key=lambda r: r[1])
                key = f"{vname}_after{after}"
                res[key] = {"min_us": best[0], "median_us": best[1], "p90_us": best[2], "max_us": best[3]}
                log(f"[bench]   first load {vname:12s} with {after} behind: min {best[0]:.2f} median {best[1]:.2f} "
                    f"p90 {best[2]:.2f} max {best[3]:.2f} us")
        print(json.dumps({"first_load_latency": res}), flush=True)
        dev.close()
        return
    if args.gemm_bench:
        print(json.dumps({"gemm_bench_matrix": gemm_bench_matrix(dev, m)}), flush=True)
        dev.close()
        return
    if args.attention_only or args.gemm_only or args.token_only:
        extra = {}
        if args.token_only:
            token_extras(dev, m, max(10, args.steps // 2), 3, extra)
        if args.gemm_only:
            gemm_extras(dev, m, 20, 5, extra)
        if args.attention_only:
            f4_extras(dev, m, 20, 5, extra)
        dev.close()
        print(json.dumps({"workloads": extra}), flush=True)
        return

    log("[bench] headline: phi15 decode step, Q8_0, M=1")
    head = decode_step(dev, m, "q8_0", 1, args.steps, args.warmup, graph=not args.eager)
    log(f"[bench]   {head['ms_per_step'] * 1e3:.1f} us/step  {head['gbs']:.0f} GB/s ({100 * head['frac']:.1f}% of "
        f"8 TB/s); kernel-time sum {head['kernel_ms_sum'] * 1e3:.1f} us -> {head['kernel_gbs']:.0f} GB/s")

    extra = {}
    if not args.quick:
        for qt, M, grp in (("q8_0", 1, False), ("q4_0", 1, True), ("q4_0", 1, False), ("q4_0", 4, True),
                           ("q4_0", 16, True), ("q8_0", 4, True)):
            r = decode_step(dev, m, qt, M, max(10, args.steps // 2), 3, grouped=grp)
            extra[r["workload"]] = r
            log(f"[bench]   {r['workload']}: {r['ms_per_step'] * 1e3:.1f} us/step {r['gbs']:.0f} GB/s "
                f"({100 * r['frac']:.1f}%)")
        token_extras(dev, m, max(10, args.steps // 2), 3, extra)
        r = fp32_gemv(dev, m, max(10, args.steps // 2), 3)
        extra[r["workload"]] = r
        log(f"[bench]   {r['workload']}: {r['us']:.1f} us {r['gbs']:.0f} GB/s ({100 * r['frac']:.1f}%)")
        r = gemv_exact(dev, m, 32, 4)
        extra[r["workload"]] = r
        log(f"[bench]   {r['workload']}: {r['kernel_us']:.1f} us kernel {r['gbs']:.0f} GB/s "
            f"({100 * r['frac']:.1f}%; reference summation order)")
        gemm_extras(dev, m, 20, 5, extra)
        f4_extras(dev, m, 20, 5, extra)
        log("[bench] gemm_bench.cpp's variant x config table")
        extra["gemm_bench_matrix"] = gemm_bench_matrix(dev, m)

    cpu = None
    if not args.no_cpu:
        log("[bench] CPU baseline (oracle Q8_0 GEMV on host cores)")
        cpu = cpu_baseline(args.cpu_seconds)
        log(f"[bench]   {cpu['value']:.2f} GB/s on {cpu['cores']} threads, {cpu['single_thread_value']:.2f} GB/s on 1")
        for leg in cpu["legs"]:
            log(f"[bench]   cpu {leg['kernel']} {leg['shape']} on {leg['threads']} threads: "
                + (f"{leg['gbs']:.2f} GB/s" if "gbs" in leg else f"{leg['gflops']:.2f} GFLOP/s"))
    dev.close()

    out = {
        "metric": "decode GEMV HBM GB/s (Q8_0, Phi-1.5 decode step, M=1)",
        "value": round(head["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (SplitMix64/Box-Muller seeded Q8_0 blocks: qs uniform [-127,127], "
                "d=f16(|N(0,0.02)|/127); x ~ N(0,1) fp32)",
        "config": {"workload": "phi15_decode_q8_0", "model": "Phi-1.5 weight set (24 layers, d=2048, ffn 8192, "
                   "vocab 51200)", "gemvs_per_step": 97, "launches_per_step": head["launches"], "M": 1,
                   "weight_format": "GGUF Q8_0 (packed split)",
                   "bytes_per_step": head["bytes_per_step"], "graph": not args.eager,
                   "grouping": "per layer {QKV, fc1} and {dense, fc2} as one launch each (independent in "
                               "Phi-1.5's parallel block); LM head alone",
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(head["gbs"], 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(head["frac"], 4), "traffic": measured_traffic(),
                     "peak_box": round(BOX_PEAK["hbm"], 1), "frac_box": round(head["gbs"] / BOX_PEAK["hbm"], 4),
                     "peak_note": "peak = MI355X nominal 8 TB/s; peak_box = this device's memory clock x bus "
                                  "width x 4 / 8 (HBM3E, mvlm_device_info)",
                     "traffic_note": "HBM bytes per step (49 launches) from rocprofv3 FETCH_SIZE + WRITE_SIZE, "
                                     "scaled by a 256 MiB device copy; " + os.path.relpath(TRAFFIC_FILE, ROOT),
                     "kernel": "gemv_stream_kernel<Q8Fmt>",
                     "timing": f"algorithmic bytes of one step / ({head['launches']} x the kernel's average "
                               "launch duration), the average being the timed region (HIP events on the plan's "
                               "stream around the graph replays) divided by the launches it holds (every launch "
                               "of the step is this kernel)",
                     "kernel_events_us_per_step": round(head["kernel_ms_sum"] * 1e3, 2),
                     "kernel_events_frac": round(head["kernel_frac"], 4),
                     "kernel_events_note": "sum of the 49 kernel execution times from HIP start/stop events on "
                                           "each launch's own dispatch packet, median of 5 eager steps (no "
                                           "inter-launch gaps)"},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
