"""Pins the CPU oracle (oracle/oracle.c) before anything is checked against it.

Each restated function meets at least one check that does not retype its
formula: committed golden fixtures, numpy's independent float16 conversion,
exact-integer cases where every summation order agrees bit for bit, closed
forms (one-hot, identity), fp64 brute force, and cross-checks between the
restatements of kernels that share an fma order in the reference
(gemm_naive, gemm_tiled and gemm_image, src/kernels/gemm.cl:26-200).
"""
import json
import os

import numpy as np
import pytest

from conftest import within

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load_blocks():
    with open(os.path.join(GOLDEN, "blocks_known_answer.json")) as f:
        return json.load(f)


# ---- number formats ----------------------------------------------------------

def test_f16_rne_matches_numpy(orc):
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2 ** 32, 400_000, dtype=np.uint64).astype(np.uint32)
    # add every boundary neighbourhood: ties, subnormal edge, overflow edge
    edges = np.array([0x33000000, 0x33000001, 0x387FE000, 0x38800000, 0x477FEFFF, 0x477FF000,
                      0x3F801000, 0x3F803000, 0x7F800000, 0x00000001], np.uint32)
    bits = np.concatenate([bits, edges, edges | 0x80000000])
    f = bits.view(np.float32)
    mine = orc.f32_to_f16(f)
    with np.errstate(over="ignore"):
        ref = f.astype(np.float16).view(np.uint16)
    finite = ~np.isnan(f)
    assert np.array_equal(mine[finite], ref[finite])
    assert np.all(np.isnan(orc.f16_to_f32(mine[~finite])))


def test_f16_widen_all_patterns(orc):
    allh = np.arange(65536, dtype=np.uint16)
    mine = orc.f16_to_f32(allh)
    ref = allh.view(np.float16).astype(np.float32)
    same = (mine.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(mine) & np.isnan(ref))
    assert same.all()


def test_bf16_rne(orc):
    # every bf16 value round-trips; the midpoint between two neighbours rounds to the even one
    allb = np.arange(65536, dtype=np.uint16)
    f = orc.bf16_to_f32(allb)
    fin = ~np.isnan(f)
    assert np.array_equal(orc.f32_to_bf16(f[fin]), allb[fin])
    lo = np.arange(0x3F80, 0x3FA0, dtype=np.uint32)
    mid = ((lo << 16) | 0x8000).view(np.float32)
    expect = np.where(lo % 2 == 0, lo, lo + 1).astype(np.uint16)
    assert np.array_equal(orc.f32_to_bf16(mid), expect)
    above = ((lo << 16) | 0x8001).view(np.float32)
    assert np.array_equal(orc.f32_to_bf16(above), (lo + 1).astype(np.uint16))


# ---- GGUF blocks ---------------------------------------------------------------

def test_block_sizes_match_reference_tests(orc):
    """tests/test_gguf.cpp:16-34 of the reference: F32 4, F16 2, Q4_0 18, Q8_0 34; blocks of 32."""
    g = load_blocks()
    ids = {"F32": 0, "F16": 1, "Q4_0": 2, "Q8_0": 8}
    for name, tid in ids.items():
        assert orc.lib().orc_ggml_type_size(tid) == g["type_sizes"][name]
        assert orc.lib().orc_ggml_block_size(tid) == g["block_sizes"][name]


def test_dequant_known_answer_blocks(orc):
    for case in load_blocks()["cases"]:
        raw = np.frombuffer(bytes.fromhex(case["bytes"]), np.uint8).copy()
        out = orc.dequant_q8_0(raw) if case["type"] == "q8_0" else orc.dequant_q4_0(raw)
        assert np.array_equal(out.view(np.uint32), np.array(case["bits"], np.uint32)), case["name"]


def test_dequant_matches_brute_force_definition(orc):
    """Random blocks against the definition evaluated in fp64 with numpy's fp16 decoding."""
    nb = 500
    q8 = orc.q8_0_blocks(nb, 11)
    q4 = orc.q4_0_blocks(nb, 12)
    blk8 = q8.reshape(nb, 34)
    d8 = blk8[:, :2].copy().view(np.float16).astype(np.float64)
    qs8 = blk8[:, 2:].view(np.int8).astype(np.float64)
    assert np.array_equal(orc.dequant_q8_0(q8), (qs8 * d8).astype(np.float32).ravel())
    blk4 = q4.reshape(nb, 18)
    d4 = blk4[:, :2].copy().view(np.float16).astype(np.float64)
    qs4 = blk4[:, 2:].astype(np.int64)
    codes = np.concatenate([qs4 & 15, qs4 >> 4], axis=1).astype(np.float64) - 8.0
    assert np.array_equal(orc.dequant_q4_0(q4), (codes * d4).astype(np.float32).ravel())


def test_generated_block_distributions(orc):
    nb = 4000
    q8 = orc.q8_0_blocks(nb, 21).reshape(nb, 34)
    qs = q8[:, 2:].view(np.int8)
    assert qs.min() == -127 and qs.max() == 127           # never -128
    d = q8[:, :2].copy().view(np.float16).astype(np.float64)
    assert np.all(d >= 0) and abs(np.mean(d * 127) - 0.02 * np.sqrt(2 / np.pi)) < 1e-3
    q4 = orc.q4_0_blocks(nb, 22).reshape(nb, 18)
    codes = np.concatenate([q4[:, 2:] & 15, q4[:, 2:] >> 4])
    assert codes.min() == 0 and codes.max() == 15
    d4 = q4[:, :2].copy().view(np.float16).astype(np.float64)
    assert abs(np.mean(d4 * 8) - 0.02 * np.sqrt(2 / np.pi)) < 1e-3


def test_normal_generator_moments_and_determinism(orc):
    x = orc.normal_f32(200_000, orc.seed_for(1))
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1.0) < 0.01
    assert np.array_equal(x, orc.normal_f32(200_000, orc.seed_for(1)))
    assert not np.array_equal(x[:100], orc.normal_f32(100, orc.seed_for(2)))
    # counter-based: a prefix equals the first elements of a longer fill
    assert np.array_equal(orc.normal_f32(1001, 5)[:1000], orc.normal_f32(1000, 5))
    # Box-Muller pairs: even/odd elements share a radius, r^2 = x_even^2 + x_odd^2 = -2 ln u1
    u1 = np.array([orc.lib().orc_uniform_at(5, 2 * j) for j in range(50)])
    xx = orc.normal_f32(100, 5).astype(np.float64)
    assert np.allclose(xx[0::2] ** 2 + xx[1::2] ** 2, -2 * np.log(u1), rtol=1e-6)


# ---- restatements of gemm.cl ------------------------------------------------------

def golden_gemm_cases():
    z = np.load(os.path.join(GOLDEN, "gemm_exact_int.npz"))
    i = 0
    while f"case{i}_shape" in z:
        M, N, K = (int(v) for v in z[f"case{i}_shape"])
        yield M, N, K, z[f"case{i}_A"], z[f"case{i}_B"], z[f"case{i}_C16"], z[f"case{i}_C32"]
        i += 1


def test_reference_kernels_on_exact_integer_fixtures(orc):
    for M, N, K, A, B, C16, C32 in golden_gemm_cases():
        for fn in (orc.gemm_naive, orc.gemm_tiled, orc.gemm_image):
            c16, c32 = fn(A, B, M, N, K)
            assert np.array_equal(c16, C16) and np.array_equal(c32, C32)
        if M == 1:
            y16, y32 = orc.gemv(A[0], B, N, K)
            assert np.array_equal(y16, C16[0]) and np.array_equal(y32, C32[0])


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (5, 9, 17), (13, 37, 45), (16, 16, 64), (3, 70, 300)])
def test_naive_tiled_image_share_fma_order(orc, M, N, K):
    A = orc.normal_f16(M * K, 31)
    B = orc.normal_f16(K * N, 32, 0.02)
    n16, n32 = orc.gemm_naive(A, B, M, N, K)
    for fn in (orc.gemm_tiled, orc.gemm_image):
        c16, c32 = fn(A, B, M, N, K)
        assert np.array_equal(c16, n16) and np.array_equal(c32.view(np.uint32), n32.view(np.uint32))


def test_gemv_against_fp64_and_naive(orc):
    N, K = 67, 1000
    x = orc.normal_f16(K, 41)
    B = orc.normal_f16(K * N, 42, 0.02)
    y16, y32 = orc.gemv(x, B, N, K)
    xf = orc.f16_to_f32(x).astype(np.float64)[None, :]
    Bf = orc.f16_to_f32(B).astype(np.float64).reshape(K, N)
    ref, scale = orc.gemm_f64(xf, Bf.T.copy(), 1, N, K)
    ok, worst = within(y32, ref[0], scale[0], 1e-6)
    assert ok, worst
    # the stored fp16 is the RNE rounding of the fp32 accumulator
    assert np.array_equal(y16, orc.f32_to_f16(y32))
    # a different partition of the same sum (tree vs chain) differs only by rounding
    _, n32 = orc.gemm_naive(x, B, 1, N, K)
    assert within(y32, n32[0], scale[0], 1e-6)[0]


def test_threaded_reference_kernels_are_bit_identical(orc):
    """orc_gemv_mt / orc_gemm_image_mt (the host baseline's threaded runs) give
    the single-thread restatement's bits"""
    M, N, K = 9, 70, 300
    A = orc.normal_f16(M * K, 61)
    B = orc.normal_f16(K * N, 62, 0.02)
    c16, c32 = orc.gemm_image(A, B, M, N, K)
    t16, t32 = orc.gemm_image_mt(A, B, M, N, K, 0)
    assert np.array_equal(c16, t16) and np.array_equal(c32.view(np.uint32), t32.view(np.uint32))
    y16, y32 = orc.gemv(A[:K], B, N, K)
    z16, z32 = orc.gemv(A[:K], B, N, K, nthreads=0)
    assert np.array_equal(y16, z16) and np.array_equal(y32.view(np.uint32), z32.view(np.uint32))


def gemv_fold_cases():
    path = os.path.join(os.path.dirname(__file__), "golden", "gemv_fold_order.json")
    return json.load(open(path))["cases"]


@pytest.mark.parametrize("case", gemv_fold_cases(), ids=lambda c: c["name"])
def test_gemv_summation_order_fixture(orc, case):
    """Hand-built inputs whose fp16 result only the reference gemv's order gives
    (strided k partition, ascending k per work item, fold pairs 128..1;
    tests/golden/make_gemv_fold_fixture.py derives each expected value)"""
    K, N = case["K"], case["N"]
    x = np.array(case["x"], np.uint16)
    W = np.array(case["W_kn"], np.uint16)
    y16, _ = orc.gemv(x, W, N, K)
    assert y16.tolist() == case["y_bits"], case["name"]
    assert case["y_bits"] != case["other_bits"]          # the case separates the two orders


def test_closed_forms(orc):
    K, N = 96, 40
    B = orc.normal_f16(K * N, 51, 0.5)
    for k in (0, 17, 95):
        x = np.zeros(K, np.uint16)
        x[k] = 0x3C00  # 1.0
        y16, y32 = orc.gemv(x, B, N, K)
        assert np.array_equal(y16, B.reshape(K, N)[k])
        c16, _ = orc.gemm_naive(x, B, 1, N, K)
        assert np.array_equal(c16[0], B.reshape(K, N)[k])
    eye = np.eye(K, dtype=np.float16).view(np.uint16)
    A = orc.normal_f16(7 * K, 52)
    c16, _ = orc.gemm_tiled(A, eye, 7, K, K)
    assert np.array_equal(c16, A.reshape(7, K))


# ---- the NT path -------------------------------------------------------------------

@pytest.mark.parametrize("kind", ["f32", "f16", "bf16", "q8_0", "q4_0"])
def test_nt_gemm_against_fp64(orc, kind):
    M, N, K = 3, 45, 256
    if kind == "f32":
        X = orc.normal_f32(M * K, 61); W = orc.normal_f32(N * K, 62, 0.02)
        Xf, Wf = X.astype(np.float64), W.astype(np.float64)
    elif kind in ("f16", "bf16"):
        gen, wid = (orc.normal_f16, orc.f16_to_f32) if kind == "f16" else (orc.normal_bf16, orc.bf16_to_f32)
        X = gen(M * K, 61); W = gen(N * K, 62, 0.02)
        Xf, Wf = wid(X).astype(np.float64), wid(W).astype(np.float64)
    else:
        X = orc.normal_f32(M * K, 61)
        W = orc.q8_0_blocks(N * K // 32, 62) if kind == "q8_0" else orc.q4_0_blocks(N * K // 32, 62)
        deq = orc.dequant_q8_0 if kind == "q8_0" else orc.dequant_q4_0
        Xf, Wf = X.astype(np.float64), deq(W).astype(np.float64)
    Y = orc.gemm_nk(kind, X, W, M, N, K)
    ref, scale = orc.gemm_f64(Xf.reshape(M, K), Wf.reshape(N, K), M, N, K)
    ok, worst = within(Y, ref, scale, 1e-6)
    assert ok, worst
    # the thread count does not change any bit
    assert np.array_equal(Y, orc.gemm_nk(kind, X, W, M, N, K, nthreads=1))


def test_nt_gemm_is_transposed_reference_gemm(orc):
    """The NT restatement of an fp16 product equals gemm_naive's fp32 accumulator on W^T:
    same operands, same ascending-k fma chain."""
    M, N, K = 4, 24, 130
    X = orc.normal_f16(M * K, 71)
    W = orc.normal_f16(N * K, 72, 0.02)
    WT = W.reshape(N, K).T.copy()
    _, n32 = orc.gemm_naive(X, WT, M, N, K)
    Y = orc.gemm_nk("f16", X, W, M, N, K)
    assert np.array_equal(Y.view(np.uint32), n32.view(np.uint32))


def test_batched_against_per_head_products(orc):
    H, S, D = 3, 19, 24
    Q = orc.normal_f16(S * H * D, 81)
    Kt = orc.normal_f16(S * H * D, 82)
    C = orc.gemm_batched_f16(Q, Kt, H, S, S, D, H * D, H * D, S, D, D, S * S, H * S * S)
    for h in range(H):
        q = Q.reshape(S, H, D)[:, h, :].copy()
        k = Kt.reshape(S, H, D)[:, h, :].copy()
        ref = orc.gemm_nk("f16", q, k, S, S, D)
        assert np.array_equal(C.reshape(H, S, S)[h], ref)


# ---- fused epilogue (activations.cl formulas) ------------------------------

def test_gelu_tanh_pins(orc):
    from scipy.special import erf
    g = orc.lib().orc_gelu_tanh
    xs = np.linspace(-6.0, 6.0, 1201)
    vals = np.array([g(float(x)) for x in xs])
    assert g(0.0) == 0.0
    # the tanh form is exactly x-odd-symmetric: gelu(x) - gelu(-x) = x
    assert np.allclose(vals - vals[::-1], xs, rtol=0, atol=1e-12)
    # within the tanh approximation's known distance of the erf GELU
    # (a dropped cubic term or a wrong sqrt(2/pi) would exceed 1e-3)
    exact = 0.5 * xs * (1.0 + erf(xs / np.sqrt(2.0)))
    assert np.max(np.abs(vals - exact)) < 1e-3
    assert abs(g(20.0) - 20.0) < 1e-12 and abs(g(-20.0)) < 1e-12


def test_silu_pins(orc):
    s = orc.lib().orc_silu
    assert s(0.0) == 0.0
    for x in (0.1, 1.0, 3.7, 15.0):
        assert abs((s(x) - s(-x)) - x) < 1e-12          # x sigma(x) + x sigma(-x) = x
    assert abs(s(np.log(3.0)) - 0.75 * np.log(3.0)) < 1e-15


def test_epilogue_order(orc):
    # act(acc + bias) * mul + res, bias per column, mul/res per element
    Y = np.array([[1.0, -2.0, 0.0]])
    out = orc.epilogue_f64(Y, bias=[0.5, 2.0, -1.0], mul=[[2.0, 3.0, 4.0]], res=[[10.0, 20.0, 30.0]], act=2)
    sil = orc.lib().orc_silu
    assert np.allclose(out, [[sil(1.5) * 2 + 10, sil(0.0) * 3 + 20, sil(-1.0) * 4 + 30]], rtol=0, atol=1e-15)
    assert np.array_equal(orc.epilogue_f64(Y), Y)


# ---- attention (attention.cl:46-179 prefill, :197-295 decode) ----------------

def _f16(x):
    """fp16 bits of x by numpy's own RNE conversion, and the values they hold."""
    bits = np.asarray(x, np.float16).view(np.uint16)
    return bits, bits.view(np.float16).astype(np.float64)


@pytest.mark.parametrize("causal", [False, True])
def test_attention_constant_values(orc, causal):
    # V constant along the keys: every convex combination returns it
    rng = np.random.default_rng(11)
    Sq, Skv, H, D = 7, 13, 3, 16
    Q, _ = _f16(rng.standard_normal((Sq, H, D)))
    K, _ = _f16(rng.standard_normal((Skv, H, D)))
    c = rng.standard_normal((H, D))
    V, cv = _f16(np.broadcast_to(c, (Skv, H, D)))
    O, A, _ = orc.attention_f64(Q, K, V, Sq, Skv, H, D, causal)
    assert np.allclose(O, np.broadcast_to(cv[0], O.shape), rtol=1e-14, atol=0)
    assert np.allclose(A, np.abs(O), rtol=1e-14, atol=0)


def test_attention_zero_query_is_running_mean(orc):
    # Q = 0: all visible scores equal, so O is the mean of the visible V rows.
    # Causal with seq_q < seq_kv: query i sees keys 0 .. i + (seq_kv - seq_q).
    rng = np.random.default_rng(12)
    Sq, Skv, H, D = 5, 9, 2, 8
    Q, _ = _f16(np.zeros((Sq, H, D)))
    K, _ = _f16(rng.standard_normal((Skv, H, D)))
    V, v = _f16(rng.standard_normal((Skv, H, D)))
    O, _, _ = orc.attention_f64(Q, K, V, Sq, Skv, H, D, causal=False)
    assert np.allclose(O, np.broadcast_to(v.mean(axis=0), O.shape), rtol=0, atol=1e-14)
    O, _, _ = orc.attention_f64(Q, K, V, Sq, Skv, H, D, causal=True)
    running = np.cumsum(v, axis=0) / np.arange(1, Skv + 1)[:, None, None]
    assert np.allclose(O, running[Skv - Sq:], rtol=0, atol=1e-14)


def test_attention_causal_first_query_is_first_value(orc):
    rng = np.random.default_rng(13)
    S, H, D = 6, 4, 24
    Q, _ = _f16(rng.standard_normal((S, H, D)))
    K, _ = _f16(rng.standard_normal((S, H, D)))
    V, v = _f16(rng.standard_normal((S, H, D)))
    O, _, _ = orc.attention_f64(Q, K, V, S, S, H, D, causal=True)
    assert np.array_equal(O[0], v[0])
    # the last query sees every key: same row as the unmasked product
    O2, _, _ = orc.attention_f64(Q, K, V, S, S, H, D, causal=False)
    assert np.array_equal(O[-1], O2[-1])


def test_attention_two_keys_is_a_sigmoid(orc):
    # two keys: weights sigma(s0 - s1), sigma(s1 - s0) with s = q.k / sqrt(64) = q.k / 8
    rng = np.random.default_rng(14)
    H, D = 3, 64
    Q, q = _f16(rng.standard_normal((1, H, D)))
    K, k = _f16(rng.standard_normal((2, H, D)))
    V, v = _f16(rng.standard_normal((2, H, D)))
    O, _, R = orc.attention_f64(Q, K, V, 1, 2, H, D)
    s = np.einsum("hd,khd->kh", q[0], k) / 8.0
    w0 = 1.0 / (1.0 + np.exp(s[1] - s[0]))
    want = w0[:, None] * v[0] + (1.0 - w0)[:, None] * v[1]
    assert np.allclose(O[0], want, rtol=1e-12, atol=1e-14)
    assert np.allclose(R[0], np.max(np.einsum("hd,khd->khd", q[0], k).__abs__().sum(-1), axis=0) / 8.0,
                       rtol=1e-14)
    # an explicit scale replaces 1/sqrt(D)
    O3, _, _ = orc.attention_f64(Q, K, V, 1, 2, H, D, scale=0.0)
    assert np.allclose(O3[0], 0.5 * (v[0] + v[1]), rtol=0, atol=1e-15)


def test_attention_selects_matching_key(orc):
    # one-hot keys and queries: query (i, h) matches key (3i + h) % 16 only, with
    # score 64 / sqrt(16) = 16 against 0, so O is that key's V row to within
    # 15 e^-16 of its magnitude; a transposed or head-swapped index picks another row
    H, D, Skv, Sq = 2, 16, 16, 10
    K = np.zeros((Skv, H, D))
    for k in range(Skv):
        for h in range(H):
            K[k, h, (k + 5 * h) % D] = 8.0
    Qv = np.zeros((Sq, H, D))
    match = np.zeros((Sq, H), int)
    for i in range(Sq):
        for h in range(H):
            match[i, h] = (3 * i + h) % Skv
            Qv[i, h] = K[match[i, h], h]
    Qb, _ = _f16(Qv)
    Kb, _ = _f16(K)
    rng = np.random.default_rng(15)
    V, v = _f16(rng.uniform(1.0, 2.0, (Skv, H, D)))
    O, _, _ = orc.attention_f64(Qb, Kb, V, Sq, Skv, H, D)
    for i in range(Sq):
        for h in range(H):
            assert np.allclose(O[i, h], v[match[i, h], h], rtol=15 * np.exp(-16.0) * 2, atol=0), (i, h)


def test_attention_heads_are_independent(orc):
    rng = np.random.default_rng(16)
    S, H, D = 8, 5, 8
    Q, _ = _f16(rng.standard_normal((S, H, D)))
    K, _ = _f16(rng.standard_normal((S, H, D)))
    V, _ = _f16(rng.standard_normal((S, H, D)))
    perm = rng.permutation(H)
    O, _, _ = orc.attention_f64(Q, K, V, S, S, H, D, causal=True)
    Op, _, _ = orc.attention_f64(Q[:, perm], K[:, perm], V[:, perm], S, S, H, D, causal=True)
    assert np.array_equal(Op, O[:, perm])


# ---- LM-head token pick (moondream2.cpp:553-593) ------------------------------

F32_ID, F16_ID, BF16_ID = 0, 1, 30


def _bf16_bits(v32):
    return (np.asarray(v32, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def test_argmax_distinct_values_match_numpy(orc):
    rng = np.random.default_rng(21)
    rows, n = 5, 3001
    x = rng.permutation(rows * n).astype(np.float32).reshape(rows, n) - 7000.0    # distinct, exact in fp32
    assert np.array_equal(orc.argmax(x, F32_ID, rows, n, n), np.argmax(x, axis=1))
    h = rng.permutation(2000).astype(np.float16)[:1999] - np.float16(1000)       # distinct, exact in fp16
    assert orc.argmax(h.view(np.uint16), F16_ID, 1, h.size, h.size)[0] == int(np.argmax(h))
    b = _bf16_bits(x)                                                           # ties possible: first wins
    vals = (b.astype(np.uint32) << 16).view(np.float32)
    want = [int(np.flatnonzero(r == r.max())[0]) for r in vals]
    assert orc.argmax(b, BF16_ID, rows, n, n).tolist() == want


def test_argmax_keys_and_ties(orc):
    def f16(vals):
        return np.array(vals, np.float16).view(np.uint16)
    neg_sub = np.uint16(0x8001)                              # -smallest subnormal: counts as +0
    cases = [
        (f16([1.0, 3.0, 3.0, 2.0]), 1),                      # first of equal maxima
        (f16([-np.inf, -np.inf]), 0),                        # nothing beats the start
        (f16([-1.0, np.inf, 5.0, np.inf]), 1),
        (f16([0.5, np.nan]), 1),                             # +NaN is +inf
        (np.array([0x3C00, 0xFE00], np.uint16), 0),          # -NaN is -inf
        (np.array([neg_sub, 0x0000], np.uint16), 0),         # subnormal == 0: first wins
        (np.array([0x8000, 0x0001, 0x0000], np.uint16), 0),  # -0, +subnormal, +0 all equal
        (f16([-2.0, -np.inf, -1.5]), 2),
    ]
    for bits, want in cases:
        assert orc.lib().orc_argmax_f16_reference(bits, bits.size) == want, bits
        assert orc.argmax(bits, F16_ID, 1, bits.size, bits.size)[0] == want, bits
    f = np.array([1e38, np.inf, 3.0], np.float32)
    assert orc.argmax(f, F32_ID, 1, 3, 3)[0] == 1
    f = np.array([np.float32(1e-40), 0.0, -1e-40], np.float32)   # fp32 subnormals count as 0
    assert orc.argmax(f, F32_ID, 1, 3, 3)[0] == 0


def test_argmax_generalised_key_equals_reference_scan_on_f16(orc):
    rng = np.random.default_rng(22)
    for trial in range(20):
        bits = rng.integers(0, 1 << 16, 4096, dtype=np.uint16)     # every class: NaN, inf, subnormal, ±0
        if trial % 2:
            bits[rng.integers(0, 4096, 50)] = 0x7C00
        assert orc.argmax(bits, F16_ID, 1, bits.size, bits.size)[0] == \
            orc.lib().orc_argmax_f16_reference(bits, bits.size)


def test_argmax_rows_and_stride(orc):
    rng = np.random.default_rng(23)
    x = rng.standard_normal((4, 100)).astype(np.float32)
    got = orc.argmax(x, F32_ID, 3, 60, 100)                    # 3 rows of 60, stride 100
    assert got.tolist() == np.argmax(x[:3, :60], axis=1).tolist()
