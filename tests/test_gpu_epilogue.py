"""Fused epilogues (mvlm_epilogue): out = act(acc + bias[n]) * mul + residual,
applied in the store of the MFMA GEMM, the streaming GEMV (M = 1) and the
long-row skinny path, checked against the oracle's fp64 GEMM followed by its
fp64 epilogue (oracle/oracle.c orc_epilogue_f64: the formulas of
activations.cl:22 and :68, bias as vision.cl:178-186, residual as
activations.cl:259-290).

Tolerance per element: the accumulator's bound (rtol * S, S = sum |x*w|)
carried through the activation (slope <= 1.2) and the gate factor, plus a
few fp32 ulps of the epilogue arithmetic, plus half an ulp of the output
dtype."""
from __future__ import annotations

import numpy as np
import pytest

import mvlm_amd as m
from mvlm_amd import native

pytestmark = pytest.mark.gpu

F32, F16, BF16 = m.F32, m.F16, m.BF16
NONE, GELU, SILU = native.ACT_NONE, native.ACT_GELU_TANH, native.ACT_SILU


def to_storage(orc, v32, dt):
    """fp32 values -> (bits or floats in the dtype's storage, their exact fp64 values)."""
    v32 = np.ascontiguousarray(v32, np.float32)
    if dt == F32:
        return v32, v32.astype(np.float64)
    if dt == F16:
        bits = np.empty(v32.size, np.uint16)
        orc.lib().orc_f32_to_f16_array(v32, bits, v32.size)
        back = np.empty(v32.size, np.float32)
        orc.lib().orc_f16_to_f32_array(bits, back, v32.size)
        return bits, back.astype(np.float64)
    bits = np.empty(v32.size, np.uint16)
    orc.lib().orc_f32_to_bf16_array(v32, bits, v32.size)
    back = np.empty(v32.size, np.float32)
    orc.lib().orc_bf16_to_f32_array(bits, back, v32.size)
    return bits, back.astype(np.float64)


def from_storage(orc, raw, dt):
    if dt == F32:
        return raw.astype(np.float64)
    back = np.empty(raw.size, np.float32)
    (orc.lib().orc_f16_to_f32_array if dt == F16 else orc.lib().orc_bf16_to_f32_array)(
        np.ascontiguousarray(raw, np.uint16), back, raw.size)
    return back.astype(np.float64)


def half_ulp(v, dt):
    mant = {F32: 24, F16: 11, BF16: 8}[dt]
    return np.abs(v) * 2.0 ** -mant + (6e-8 if dt == F16 else 0.0)


def make_operands(dev, orc, M, N, dt, seed, bias, mul, residual):
    rng = np.random.default_rng(seed)
    ops, vals = {}, {}
    for name, want, shape in (("bias", bias, N), ("mul", mul, M * N), ("residual", residual, M * N)):
        if want:
            raw, v = to_storage(orc, rng.standard_normal(shape).astype(np.float32), dt)
            ops[name] = dev.upload(raw)
            vals[name] = v
        else:
            ops[name] = None
            vals[name] = None
    return ops, vals


def check(orc, got, Y64, S, vals, act, dt, rtol):
    M, N = Y64.shape
    ref = orc.epilogue_f64(Y64, vals["bias"], None if vals["mul"] is None else vals["mul"].reshape(M, N),
                           None if vals["residual"] is None else vals["residual"].reshape(M, N), act)
    gate = np.ones((M, N)) if vals["mul"] is None else np.abs(vals["mul"].reshape(M, N))
    res = np.zeros((M, N)) if vals["residual"] is None else np.abs(vals["residual"].reshape(M, N))
    body = orc.epilogue_f64(Y64, vals["bias"], act=act)
    tol = rtol * S * 1.2 * gate + 4e-6 * (np.abs(body) * gate + res) + half_ulp(ref, dt) + 1e-30
    err = np.abs(got - ref)
    assert np.all(err <= tol), float(np.max(err / tol))


EPILOGUES = [(True, NONE, False, False), (True, GELU, False, False), (False, SILU, True, False),
             (True, NONE, False, True), (True, GELU, True, True), (False, SILU, False, True)]


@pytest.mark.parametrize("bias,act,mul,residual", EPILOGUES)
@pytest.mark.parametrize("cd", [F32, F16, BF16])
def test_gemm_packed_epilogue(dev, orc, bias, act, mul, residual, cd):
    M, N, K = 129, 200, 256
    A = orc.normal_f16(M * K, 0x71)
    Wt = orc.normal_f16(N * K, 0x72, 0.05)
    W = dev.pack(Wt, F16, N, K)
    ops, vals = make_operands(dev, orc, M, N, cd, 0x73, bias, mul, residual)
    dA, dC = dev.upload(A), dev.alloc(M * N * 4)
    dev.gemm_packed_ex(dA, F16, W, dC, cd, M, N, K, bias=ops["bias"], act=act, mul=ops["mul"],
                       residual=ops["residual"])
    got = from_storage(orc, dC.download(np.float32 if cd == F32 else np.uint16, M * N), cd).reshape(M, N)
    A64 = from_storage(orc, A, F16).reshape(M, K)
    W64 = from_storage(orc, Wt, F16).reshape(N, K)
    Y64, S = orc.gemm_f64(A64, W64, M, N, K)
    check(orc, got, Y64, S, vals, act, cd, 1e-4)


def test_patch_embedding_gemm_with_bias(dev, orc):
    """SigLIP's patch embedding as one GEMM: 729 patches x 588 values (3 x 14 x 14,
    K not a multiple of 8) against a 1152 x 588 weight, bias in the store, fp16
    out (moondream2.cpp:774, vision.cl:118-197)"""
    M, N, K = 729, 1152, 588
    A = orc.normal_f16(M * K, 0x91)
    Wt = orc.normal_f16(N * K, 0x92, 0.02)
    W = dev.pack(Wt, F16, N, K)
    ops, vals = make_operands(dev, orc, M, N, F16, 0x93, True, False, False)
    dC = dev.alloc(M * N * 2)
    dev.gemm_packed_ex(dev.upload(A), F16, W, dC, F16, M, N, K, bias=ops["bias"])
    got = from_storage(orc, dC.download(np.uint16, M * N), F16).reshape(M, N)
    Y64, S = orc.gemm_f64(from_storage(orc, A, F16).reshape(M, K), from_storage(orc, Wt, F16).reshape(N, K), M, N, K)
    check(orc, got, Y64, S, vals, NONE, F16, 1e-3)


def test_gemm_epilogue_residual_in_place(dev, orc):
    """residual aliasing the output: C = gelu(A W^T + b) + C"""
    M, N, K = 64, 96, 128
    A = orc.normal_f16(M * K, 0x74)
    Wt = orc.normal_f16(N * K, 0x75, 0.05)
    W = dev.pack(Wt, F16, N, K)
    ops, vals = make_operands(dev, orc, M, N, F32, 0x76, True, False, True)
    C = ops["residual"]
    dev.gemm_packed_ex(dev.upload(A), F16, W, C, F32, M, N, K, bias=ops["bias"], act=GELU, residual=C)
    got = C.download(np.float32, M * N).astype(np.float64).reshape(M, N)
    Y64, S = orc.gemm_f64(from_storage(orc, A, F16).reshape(M, K), from_storage(orc, Wt, F16).reshape(N, K), M, N, K)
    check(orc, got, Y64, S, vals, GELU, F32, 1e-4)


@pytest.mark.parametrize("qt,N,K", [(m.Q8_0, 300, 2048), (m.Q4_0, 130, 8192), (m.Q8_0, 24, 20480)])
@pytest.mark.parametrize("bias,act,mul,residual", [(True, GELU, False, False), (False, NONE, False, True),
                                                   (True, SILU, True, True)])
def test_quant_gemv_epilogue(dev, orc, qt, N, K, bias, act, mul, residual):
    """streaming GEMV stores (the 20480-long rows take the skinny path)"""
    x = orc.normal_f32(K, 0x77)
    blocks = (orc.q8_0_blocks if qt == m.Q8_0 else orc.q4_0_blocks)(N * K // 32, 0x78)
    W = dev.pack(blocks, qt, N, K)
    ops, vals = make_operands(dev, orc, 1, N, F32, 0x79, bias, mul, residual)
    y = dev.alloc(N * 4)
    dev.gemv_ex(dev.upload(x), F32, W, y, F32, N, K, bias=ops["bias"], act=act, mul=ops["mul"],
                residual=ops["residual"])
    deq = (orc.dequant_q8_0 if qt == m.Q8_0 else orc.dequant_q4_0)(blocks).astype(np.float64).reshape(N, K)
    Y64, S = orc.gemm_f64(x.astype(np.float64)[None], deq, 1, N, K)
    check(orc, y.download(np.float32).astype(np.float64)[None], Y64, S, vals, act, F32, 1e-5)


@pytest.mark.parametrize("yd", [F32, BF16])
@pytest.mark.parametrize("wd,N,K", [(F16, 515, 1024), (F16, 70, 300), (F32, 33, 4304)])
def test_dense_gemv_epilogue(dev, orc, yd, wd, N, K):
    """Streaming kernel (K=1024) and the per-wave dense kernel that takes rows the
    streaming kernel does not: F16 with K % 8 != 0, F32 rows over 16 KiB."""
    if wd == F16:
        x = orc.normal_f16(K, 0x7A)
        Wt = orc.normal_f16(N * K, 0x7B, 0.05)
        x64, W64 = from_storage(orc, x, F16), from_storage(orc, Wt, F16).reshape(N, K)
    else:
        x = orc.normal_f32(K, 0x7A)
        Wt = orc.normal_f32(N * K, 0x7B, 0.05)
        x64, W64 = x.astype(np.float64), Wt.astype(np.float64).reshape(N, K)
    W = dev.pack(Wt, wd, N, K)
    ops, vals = make_operands(dev, orc, 1, N, yd, 0x7C, True, True, True)
    y = dev.alloc(N * 4)
    dev.gemv_ex(dev.upload(x), wd, W, y, yd, N, K, bias=ops["bias"], act=GELU, mul=ops["mul"],
                residual=ops["residual"])
    got = from_storage(orc, y.download(np.float32 if yd == F32 else np.uint16, N), yd)[None]
    Y64, S = orc.gemm_f64(x64[None], W64, 1, N, K)
    check(orc, got, Y64, S, vals, GELU, yd, 1e-5)


@pytest.mark.parametrize("qt", [m.Q8_0, m.Q4_0])
@pytest.mark.parametrize("M", [1, 3, 16])
def test_grouped_epilogues(dev, orc, qt, M):
    """One grouped launch applying a different epilogue per entry, like a Phi-1.5
    block's projections: QKV + bias, fc1 + bias + GELU, dense + bias + residual,
    fc2 + bias + residual written in place.  M = 1 and 3 run the streaming kernel,
    M = 16 the skinny kernel; the plan entry gives the direct call's bits."""
    shapes = [(384, 2048, dict(bias=True)), (512, 2048, dict(bias=True, act=GELU)),
              (256, 1024, dict(bias=True, residual=True)), (130, 8192, dict(bias=True, residual=True, inplace=True))]
    deq = orc.dequant_q8_0 if qt == m.Q8_0 else orc.dequant_q4_0
    gen = orc.q8_0_blocks if qt == m.Q8_0 else orc.q4_0_blocks
    entries, eps, checks, outs = [], [], [], []
    for i, (N, K, spec) in enumerate(shapes):
        X = orc.normal_f32(M * K, 0xA0 + i)
        blocks = gen(N * K // 32, 0xB0 + i)
        W = dev.pack(blocks, qt, N, K)
        ops, vals = make_operands(dev, orc, M, N, F32, 0xC0 + i, spec.get("bias", False), False,
                                  spec.get("residual", False))
        y = ops["residual"] if spec.get("inplace") else dev.alloc(M * N * 4)
        entries.append((dev.upload(X), F32, W, y, F32))
        eps.append({"bias": ops["bias"], "act": spec.get("act", NONE), "residual": ops["residual"]})
        Y64, S = orc.gemm_f64(X.astype(np.float64).reshape(M, K), deq(blocks).astype(np.float64).reshape(N, K),
                              M, N, K)
        checks.append((Y64, S, vals, spec.get("act", NONE)))
        outs.append(y)
    # a plan copy first (in-place residual: it must read the residual before the direct call overwrites it)
    plan_outs = [dev.alloc(M * N * 4) for N, _, _ in shapes]
    plan_res = [dev.upload(e[3].download(np.float32)) if shapes[i][2].get("inplace") else None
                for i, e in enumerate(entries)]
    plan_entries = [(x, xd, W, plan_res[i] if plan_res[i] is not None else plan_outs[i], yd)
                    for i, (x, xd, W, _, yd) in enumerate(entries)]
    plan_eps = [dict(e, residual=plan_res[i]) if plan_res[i] is not None else e for i, e in enumerate(eps)]
    plan = m.Plan(dev)
    if M == 1:
        plan.add_gemv_grouped(plan_entries, epilogues=plan_eps)
        dev.gemv_grouped(entries, epilogues=eps)
    else:
        plan.add_gemm_quant_grouped(M, plan_entries, epilogues=plan_eps)
        dev.gemm_quant_grouped(M, entries, epilogues=eps)
    plan.run(1)
    dev.sync()
    for i, ((N, K, spec), y, (Y64, S, vals, act)) in enumerate(zip(shapes, outs, checks)):
        got = y.download(np.float32, M * N).astype(np.float64).reshape(M, N)
        check(orc, got, Y64, S, vals, act, F32, 1e-5)
        py = plan_res[i] if plan_res[i] is not None else plan_outs[i]
        assert np.array_equal(py.download(np.float32, M * N), y.download(np.float32, M * N)), i
    plan.destroy()


def test_plan_epilogues_match_direct_calls(dev, orc):
    M, N, K = 33, 64, 2048
    A = orc.normal_f16(M * K, 0x7D)
    Wt = orc.normal_f16(N * K, 0x7E, 0.05)
    W = dev.pack(Wt, F16, N, K)
    Wq = dev.pack(orc.q8_0_blocks(N * K // 32, 0x7F), m.Q8_0, N, K)
    x = dev.upload(orc.normal_f32(K, 0x80))
    dA = dev.upload(A)
    ops, _ = make_operands(dev, orc, M, N, F32, 0x81, True, True, True)
    c1, c2, y1, y2 = (dev.alloc(M * N * 4) for _ in range(4))
    dev.gemm_packed_ex(dA, F16, W, c1, F32, M, N, K, bias=ops["bias"], act=SILU, mul=ops["mul"],
                       residual=ops["residual"])
    dev.gemv_ex(x, F32, Wq, y1, F32, N, K, bias=ops["bias"], act=GELU)
    plan = m.Plan(dev)
    plan.add_gemm_packed_ex(dA, F16, W, c2, F32, M, bias=ops["bias"], act=SILU, mul=ops["mul"],
                            residual=ops["residual"])
    plan.add_gemv_ex(x, F32, Wq, y2, F32, bias=ops["bias"], act=GELU)
    plan.use_graph(True)
    plan.run(3)
    dev.sync()
    assert np.array_equal(c1.download(np.float32, M * N), c2.download(np.float32, M * N))
    assert np.array_equal(y1.download(np.float32, N), y2.download(np.float32, N))
    plan.destroy()


def offset_operands(dev, orc, M, N, dt, seed, offset):
    """bias, mul and residual as views starting `offset` bytes into their buffers"""
    ops, vals = make_operands(dev, orc, M, N, dt, seed, True, True, True)
    es = 4 if dt == F32 else 2
    views, parents = {}, []
    for name, n in (("bias", N), ("mul", M * N), ("residual", M * N)):
        raw = ops[name].download(np.uint8, n * es)
        parent = dev.upload(np.concatenate([np.full(offset, 0x7F, np.uint8), raw]))
        parents.append(parent)
        views[name] = parent.view(offset, n * es)
    return views, vals, parents


@pytest.mark.parametrize("yd", [F16, BF16])
def test_epilogue_operands_off_word_boundary(dev, orc, yd):
    """16-bit epilogue operands starting 2 bytes into a 32-bit word, odd N,
    through the streaming kernel (M = 1) and the MFMA GEMM"""
    N, K = 515, 1024
    x = orc.normal_f16(K, 0x81)
    Wt = orc.normal_f16(N * K, 0x82, 0.05)
    W = dev.pack(Wt, F16, N, K)
    W64 = from_storage(orc, Wt, F16).reshape(N, K)
    ops, vals, keep = offset_operands(dev, orc, 1, N, yd, 0x83, 2)
    y = dev.alloc(N * 2)
    dev.gemv_ex(dev.upload(x), F16, W, y, yd, N, K, bias=ops["bias"], act=GELU, mul=ops["mul"],
                residual=ops["residual"])
    got = from_storage(orc, y.download(np.uint16, N), yd)[None]
    Y64, S = orc.gemm_f64(from_storage(orc, x, F16)[None], W64, 1, N, K)
    check(orc, got, Y64, S, vals, GELU, yd, 1e-5)

    M = 37
    A = orc.normal_f16(M * K, 0x84)
    opsm, valsm, keepm = offset_operands(dev, orc, M, N, yd, 0x85, 2)
    C = dev.alloc(M * N * 2)
    dev.gemm_packed_ex(dev.upload(A), F16, W, C, yd, M, N, K, bias=opsm["bias"], act=SILU, mul=opsm["mul"],
                       residual=opsm["residual"])
    got = from_storage(orc, C.download(np.uint16, M * N), yd).reshape(M, N)
    Y64, S = orc.gemm_f64(from_storage(orc, A, F16).reshape(M, K), W64, M, N, K)
    check(orc, got, Y64, S, valsm, SILU, yd, 1e-4)
    for v in list(ops.values()) + list(opsm.values()):
        v.free()


def test_epilogue_argument_errors(dev, orc):
    N, K = 64, 64
    W = dev.pack(orc.normal_f16(N * K, 1), F16, N, K)
    x, y = dev.upload(orc.normal_f16(K, 2)), dev.alloc(N * 4)
    small = dev.alloc(8)
    with pytest.raises(m.MvlmError) as e:
        dev.gemv_ex(x, F16, W, y, F32, N, K, bias=small)
    assert e.value.code == native.ERR_BUFFER_TOO_SMALL
    with pytest.raises(m.MvlmError) as e:
        dev.gemv_ex(x, F16, W, y, F32, N, K, act=7)
    assert e.value.code == native.ERR_INVALID_ARG
    odd = dev.alloc(N * 4 + 4)
    for dt, es, off in ((F16, 2, 1), (F32, 4, 2)):
        y2 = dev.alloc(N * 4)
        with pytest.raises(m.MvlmError) as e:
            dev.gemv_ex(x, F16, W, y2, dt, N, K, residual=odd.view(off, N * es))
        assert e.value.code == native.ERR_INVALID_ARG and "multiple of" in str(e.value)
