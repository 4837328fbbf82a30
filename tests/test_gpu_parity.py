"""GPU parity: every entry point of the C ABI against the CPU oracle.

Bars (stated per test):
  * gemm_naive / gemm_tiled: bit-exact fp16 (same per-output fma order as the
    reference's gemm.cl:26-136 and its restatement).
  * dequantized Q8_0 / Q4_0 weights: bit-exact against the GGUF definition.
  * fp32 inputs (fp32 GEMV, dequantizing GEMV/GEMM): |y - r| <= 1e-5 * S,
    S = sum_k |x_k w_k| (fp64), r the oracle's fp32 result.
  * fp16 / bf16 inputs with fp32 accumulation: |y - r| <= 1e-3 * S, plus half
    a unit in the last place of the output type when the output is 16-bit.
"""
import numpy as np
import pytest

import mvlm_amd as m
from conftest import within

pytestmark = pytest.mark.gpu

F32, F16, BF16, Q8, Q4 = m.F32, m.F16, m.BF16, m.Q8_0, m.Q4_0


def half_ulp(v, dtype):
    v = np.abs(np.asarray(v, np.float64))
    if dtype == F32:
        return np.zeros_like(v)
    if dtype == F16:
        return 0.5 * np.spacing(v.astype(np.float16)).astype(np.float64) + 2.0 ** -25
    # bf16: 8 significant bits
    e = np.floor(np.log2(np.maximum(v, 1e-38)))
    return 0.5 * 2.0 ** (e - 7)


def widen(orc, arr, dtype):
    if dtype == F32:
        return np.asarray(arr, np.float32).astype(np.float64)
    return (orc.f16_to_f32(arr) if dtype == F16 else orc.bf16_to_f32(arr)).astype(np.float64)


def out_to_f64(orc, raw, dtype):
    return widen(orc, raw, dtype)


def gen(orc, dtype, n, seed, std=1.0):
    if dtype == F32:
        return orc.normal_f32(n, seed, std)
    return orc.normal_f16(n, seed, std) if dtype == F16 else orc.normal_bf16(n, seed, std)


def np_dtype(dtype):
    return np.float32 if dtype == F32 else np.uint16


# ---------------------------------------------------------------------------
# reference-arithmetic GEMMs: bit-exact
# ---------------------------------------------------------------------------

REF_SHAPES = [(1, 1, 1), (1, 8192, 2048), (3, 5, 7), (17, 33, 9), (64, 64, 64), (65, 130, 100),
              (32, 2048, 2048), (129, 70, 257)]


@pytest.mark.parametrize("M,N,K", REF_SHAPES)
def test_gemm_naive_and_tiled_bit_exact(dev, orc, M, N, K):
    A = orc.normal_f16(M * K, 101)
    B = orc.normal_f16(K * N, 102, 0.02)
    ref16 = (orc.gemm_naive(A, B, M, N, K)[0] if M * N * K <= 2e6 else
             orc.f32_to_f16(orc.gemm_nk("f16", A, B.reshape(K, N).T.copy(), M, N, K)))
    dA, dB = dev.upload(A), dev.upload(B)
    for fn in (dev.gemm_naive, dev.gemm_tiled):
        dC = dev.alloc(M * N * 2)
        fn(dA, dB, dC, M, N, K)
        got = dC.download(np.uint16)
        assert np.array_equal(got, ref16.ravel()), (fn.__name__, int(np.sum(got != ref16.ravel())))


def test_reference_gemms_on_exact_integer_fixtures(dev, orc):
    from test_oracle import golden_gemm_cases
    for M, N, K, A, B, C16, _ in golden_gemm_cases():
        dA, dB = dev.upload(A), dev.upload(B)
        for fn in (dev.gemm_naive, dev.gemm_tiled):
            dC = dev.alloc(M * N * 2)
            fn(dA, dB, dC, M, N, K)
            assert np.array_equal(dC.download(np.uint16), C16.ravel())
        # the same integers through the packed MFMA path and the GEMV are exact too
        W = dev.pack(B, F16, N, K, layout=m.LAYOUT_KN)
        dC = dev.alloc(M * N * 4)
        dev.gemm_packed(dA, F16, W, dC, F32, M, N, K)
        assert np.array_equal(dC.download(np.float32), C16.view(np.float16).astype(np.float32).ravel())
        if M == 1:
            y = dev.alloc(N * 2)
            dev.gemv(dA, F16, W, y, F16, N, K)
            assert np.array_equal(y.download(np.uint16), C16.ravel())
            y = dev.alloc(N * 2)
            dev.gemv_exact(dA, W, y, N, K)
            assert np.array_equal(y.download(np.uint16), C16.ravel())


# ---------------------------------------------------------------------------
# dense GEMV
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("N,K", [(8192, 2048), (1, 1), (7, 3), (130, 1000), (2048, 8192), (51200, 2048)])
def test_gemv_fp32(dev, orc, N, K):
    """fp32 x, W, y (the fp32 GEMV of benchmarks/gemm_bench.cpp's llm_ffn shape): 1e-5 * S."""
    x = orc.normal_f32(K, 111)
    W = orc.normal_f32(N * K, 112, 0.02)
    ref = orc.gemm_nk("f32", x, W, 1, N, K)[0]
    _, S = orc.gemm_f64(x.astype(np.float64)[None], W.astype(np.float64).reshape(N, K), 1, N, K)
    dW = dev.pack(W, F32, N, K)
    dx, dy = dev.upload(x), dev.alloc(N * 4)
    dev.gemv(dx, F32, dW, dy, F32, N, K)
    ok, worst = within(dy.download(np.float32), ref, S[0], 1e-5)
    assert ok, worst


@pytest.mark.parametrize("wd,xd,yd", [(F16, F16, F16), (F16, F32, F32), (BF16, BF16, F32), (BF16, F32, BF16),
                                      (F32, F16, F32)])
@pytest.mark.parametrize("N,K", [(2048, 2048), (70, 300), (5, 8)])
def test_gemv_dtypes(dev, orc, wd, xd, yd, N, K):
    x = gen(orc, xd, K, 121)
    Wt = gen(orc, wd, N * K, 122, 0.02)
    xf, Wf = widen(orc, x, xd), widen(orc, Wt, wd).reshape(N, K)
    ref, S = orc.gemm_f64(xf[None], Wf, 1, N, K)
    dW = dev.pack(Wt, wd, N, K)
    dx, dy = dev.upload(x), dev.alloc(N * 4)
    dev.gemv(dx, xd, dW, dy, yd, N, K)
    got = out_to_f64(orc, dy.download(np_dtype(yd), N), yd)
    rtol = 1e-5 if (xd == F32 and wd == F32) else 1e-3
    ok, worst = within(got, ref[0], S[0], rtol, half_ulp(ref[0], yd))
    assert ok, worst


@pytest.mark.parametrize("N,K", [(8192, 2048), (2048, 2048), (6, 300)])
def test_gemv_reference_mode_matches_restated_gemv(dev, orc, N, K):
    """fp16 x, fp16 W given as [K,N] like create_weight_image, fp16 y: the reference
    gemv (gemm.cl:219-270) restated, compared within 1e-3 * S plus half an fp16 ulp."""
    x = orc.normal_f16(K, 131)
    B = orc.normal_f16(K * N, 132, 0.02)
    ref16, ref32 = orc.gemv(x, B, N, K)
    _, S = orc.gemm_f64(orc.f16_to_f32(x).astype(np.float64)[None],
                        orc.f16_to_f32(B).astype(np.float64).reshape(K, N).T.copy(), 1, N, K)
    W = dev.pack(B, F16, N, K, layout=m.LAYOUT_KN)
    dx, dy = dev.upload(x), dev.alloc(N * 2)
    dev.gemv(dx, F16, W, dy, F16, N, K)
    got = orc.f16_to_f32(dy.download(np.uint16)).astype(np.float64)
    ok, worst = within(got, ref32, S[0], 1e-3, half_ulp(ref32, F16))
    assert ok, worst
    # the great majority of outputs round to the very same fp16 as the reference
    assert np.mean(dy.download(np.uint16) == ref16) > 0.95


@pytest.mark.parametrize("N,K", [(8192, 2048), (2048, 8192), (6, 300), (37, 1), (4099, 513), (33, 256),
                                 (130, 1000), (3, 2304), (51200, 64)])
def test_gemv_exact_bit_exact(dev, orc, N, K):
    """mvlm_gemv_exact keeps gemv's 256-partial split and fold (gemm.cl:219-270):
    every fp16 output equals the restated gemv's bit for bit, ragged N and K
    included (K = 2304 runs 8 windows together and one alone)."""
    x = orc.normal_f16(K, 141)
    B = orc.normal_f16(K * N, 142, 0.02)
    ref16, _ = orc.gemv(x, B, N, K)
    W = dev.pack(B, F16, N, K, layout=m.LAYOUT_KN)
    dx, dy = dev.upload(x), dev.alloc(N * 2)
    dev.gemv_exact(dx, W, dy, N, K)
    got = dy.download(np.uint16)
    assert np.array_equal(got, ref16), int(np.sum(got != ref16))


def test_gemv_exact_summation_order_fixture(dev):
    """the hand-built fold-order cases (tests/golden/gemv_fold_order.json): only
    the reference gemv's k partition, per-item order and fold pairs give these bits"""
    import json
    import os
    path = os.path.join(os.path.dirname(__file__), "golden", "gemv_fold_order.json")
    for case in json.load(open(path))["cases"]:
        K, N = case["K"], case["N"]
        W = dev.pack(np.array(case["W_kn"], np.uint16), F16, N, K, layout=m.LAYOUT_KN)
        x = dev.upload(np.array(case["x"], np.uint16))
        y = dev.alloc(N * 2)
        dev.gemv_exact(x, W, y, N, K)
        assert y.download(np.uint16).tolist() == case["y_bits"], case["name"]


def test_gemv_exact_errors(dev, orc):
    B = orc.normal_f16(32 * 8, 143)
    W = dev.pack(B, F16, 8, 32, layout=m.LAYOUT_KN)
    x, y = dev.alloc(64 * 2), dev.alloc(8 * 2)
    with pytest.raises(m.MvlmError):
        dev.gemv_exact(x, W, y, 8, 64)          # W is [8 x 32]
    with pytest.raises(m.MvlmError):
        dev.gemv_exact(x, W, dev.alloc(4 * 2), 8, 32)   # y holds 4 outputs
    with pytest.raises(m.MvlmError):
        dev.gemv_exact(x, dev.pack(B, BF16, 8, 32, layout=m.LAYOUT_KN), y, 8, 32)
    view = x.view(2, 64)                        # 2-byte offset: x must be 8-byte aligned
    with pytest.raises(m.MvlmError):
        dev.gemv_exact(view, W, y, 8, 32)


# ---------------------------------------------------------------------------
# quantized weights
# ---------------------------------------------------------------------------

def make_quant(orc, qt, N, K, seed):
    nb = N * K // 32
    return orc.q8_0_blocks(nb, seed) if qt == Q8 else orc.q4_0_blocks(nb, seed)


@pytest.mark.parametrize("qt", [Q8, Q4])
@pytest.mark.parametrize("N,K", [(6144, 2048), (3, 32), (50, 96)])
def test_dequant_bit_exact(dev, orc, qt, N, K):
    blocks = make_quant(orc, qt, N, K, 141)
    ref = (orc.dequant_q8_0 if qt == Q8 else orc.dequant_q4_0)(blocks).reshape(N, K)
    W = dev.pack(blocks, qt, N, K)
    got = W.dequant()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_dequant_known_answer_blocks(dev):
    import json, os
    path = os.path.join(os.path.dirname(__file__), "golden", "blocks_known_answer.json")
    for case in json.load(open(path))["cases"]:
        raw = np.frombuffer(bytes.fromhex(case["bytes"]), np.uint8).copy()
        W = dev.pack(raw, Q8 if case["type"] == "q8_0" else Q4, 1, 32)
        assert np.array_equal(W.dequant().ravel().view(np.uint32), np.array(case["bits"], np.uint32)), case["name"]


# (2048, 2048) Q8_0, (2048, 4096) and (300, 3072) Q4_0 have 2 KiB rows with
# too few rows to give every CU a block at two rows per wave: they take the
# one-row-per-wave work shape
QSHAPES = [(6144, 2048), (2048, 8192), (1, 32), (37, 96), (8192, 2048), (3456, 1152), (51200, 2048),
           (24, 20480), (5, 64), (2048, 2048), (2048, 4096), (300, 3072)]


@pytest.mark.parametrize("qt", [Q8, Q4])
@pytest.mark.parametrize("N,K", QSHAPES)
def test_quant_gemv(dev, orc, qt, N, K):
    x = orc.normal_f32(K, 151)
    blocks = make_quant(orc, qt, N, K, 152)
    kind = "q8_0" if qt == Q8 else "q4_0"
    ref = orc.gemm_nk(kind, x, blocks, 1, N, K)[0]
    deq = (orc.dequant_q8_0 if qt == Q8 else orc.dequant_q4_0)(blocks).astype(np.float64).reshape(N, K)
    _, S = orc.gemm_f64(x.astype(np.float64)[None], deq, 1, N, K)
    W = dev.pack(blocks, qt, N, K)
    dx, dy = dev.upload(x), dev.alloc(N * 4)
    (dev.gemv_q8_0 if qt == Q8 else dev.gemv_q4_0)(dx, W, dy, N, K)
    ok, worst = within(dy.download(np.float32), ref, S[0], 1e-5)
    assert ok, worst
    # the generic gemv entry (dispatch_gemv) serves quantized weights too
    dy2 = dev.alloc(N * 4)
    dev.gemv(dx, F32, W, dy2, F32, N, K)
    assert np.array_equal(dy2.download(np.float32), dy.download(np.float32))


@pytest.mark.parametrize("qt", [Q8, Q4])
@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 11, 16])
def test_quant_skinny_gemm(dev, orc, qt, M):
    N, K = 2048, 2048
    X = orc.normal_f32(M * K, 161)
    blocks = make_quant(orc, qt, N, K, 162)
    kind = "q8_0" if qt == Q8 else "q4_0"
    ref = orc.gemm_nk(kind, X, blocks, M, N, K)
    deq = (orc.dequant_q8_0 if qt == Q8 else orc.dequant_q4_0)(blocks).astype(np.float64).reshape(N, K)
    _, S = orc.gemm_f64(X.astype(np.float64).reshape(M, K), deq, M, N, K)
    W = dev.pack(blocks, qt, N, K)
    dX, dY = dev.upload(X), dev.alloc(M * N * 4)
    dev.gemm_quant(dX, W, dY, M, N, K)
    ok, worst = within(dY.download(np.float32).reshape(M, N), ref, S, 1e-5)
    assert ok, worst


@pytest.mark.parametrize("qt", [Q8, Q4])
@pytest.mark.parametrize("M,N,K,xscale", [(4, 33, 32, 1.0), (16, 17, 96, 1.0), (3, 130, 8192, 1.0),
                                          (16, 6144, 2048, 1.0), (7, 300, 2048, 3.0e4), (9, 64, 1024, 1.0e-6),
                                          (2, 51, 23 * 32, 1.0), (5, 8200, 96, 1.0), (16, 16400, 64, 1.0),
                                          (16, 12300, 2048, 1.0), (6, 16384, 64, 1.0), (11, 13000, 8192, 1.0)])
def test_quant_skinny_shapes(dev, orc, qt, M, N, K, xscale):
    # ragged N (not a multiple of the 16-row MFMA tile), fewer K blocks than
    # waves, long rows, x far from unit scale (the bf16 three-way split of x
    # must keep fp32 precision over fp32's range), and N large enough for the
    # blocks with 2 and 4 row groups per wave (ragged in the last block; 769
    # to 1024 row groups take the four-group shape with its two-block steps)
    X = (orc.normal_f32(M * K, 171) * np.float32(xscale)).astype(np.float32)
    blocks = make_quant(orc, qt, N, K, 172)
    kind = "q8_0" if qt == Q8 else "q4_0"
    ref = orc.gemm_nk(kind, X, blocks, M, N, K)
    deq = (orc.dequant_q8_0 if qt == Q8 else orc.dequant_q4_0)(blocks).astype(np.float64).reshape(N, K)
    _, S = orc.gemm_f64(X.astype(np.float64).reshape(M, K), deq, M, N, K)
    W = dev.pack(blocks, qt, N, K)
    dX, dY = dev.upload(X), dev.alloc(M * N * 4)
    dev.gemm_quant(dX, W, dY, M, N, K)
    ok, worst = within(dY.download(np.float32).reshape(M, N), ref, S, 1e-5)
    assert ok, worst


def test_weight_random_matches_oracle_generator(dev, orc):
    N, K, seed = 64, 256, 0x1234
    for qt in (Q8, Q4):
        W = dev.random_weight(qt, N, K, seed, 0.02)
        blocks = make_quant(orc, qt, N, K, seed)
        ref = (orc.dequant_q8_0 if qt == Q8 else orc.dequant_q4_0)(blocks).reshape(N, K)
        got = W.dequant()
        # codes are integer arithmetic (exact); scales pass through fp64 log/sin/cos,
        # whose last bit may differ between libraries, so allow one fp16 ulp in d
        same = got == ref
        assert same.mean() > 0.99
        assert np.allclose(got, ref, rtol=2 ** -10, atol=0)


def test_fill_normal_matches_oracle_generator(dev, orc):
    n = 10000
    buf = dev.alloc(n * 4)
    dev.fill_normal(buf, F32, n, 77, 1.0)
    got = buf.download(np.float32)
    ref = orc.normal_f32(n, 77)
    assert np.allclose(got, ref, rtol=1e-6, atol=1e-7)


# ---------------------------------------------------------------------------
# packed MFMA GEMM and batched QK^T
# ---------------------------------------------------------------------------

def check_packed(dev, orc, M, N, K, ab, cd, layout=m.LAYOUT_NK, rows=None, seed=171):
    A = gen(orc, ab, M * K, seed)
    Wt = gen(orc, ab, N * K, seed + 1, 0.02)
    src = Wt if layout == m.LAYOUT_NK else Wt.reshape(N, K).T.copy()
    W = dev.pack(src, ab, N, K, layout=layout)
    dA, dC = dev.upload(A), dev.alloc(M * N * 4)
    dev.gemm_packed(dA, ab, W, dC, cd, M, N, K)
    got = out_to_f64(orc, dC.download(np_dtype(cd), M * N), cd).reshape(M, N)
    sel = np.arange(M) if rows is None else np.unique(np.linspace(0, M - 1, rows).astype(int))
    Asel = A.reshape(M, K)[sel].copy()
    ref = orc.gemm_nk("f16" if ab == F16 else "bf16", Asel, Wt, len(sel), N, K)
    _, S = orc.gemm_f64(widen(orc, Asel, ab).reshape(len(sel), K), widen(orc, Wt, ab).reshape(N, K), len(sel), N, K)
    ok, worst = within(got[sel], ref, S, 1e-3, half_ulp(ref, cd))
    assert ok, worst
    return worst


@pytest.mark.parametrize("M,N,K", [(1, 1, 8), (5, 7, 16), (33, 65, 40), (129, 130, 200), (64, 128, 2048),
                                   (200, 300, 8)])
@pytest.mark.parametrize("ab,cd", [(F16, F32), (F16, F16), (BF16, F32), (BF16, BF16)])
def test_gemm_packed_small(dev, orc, M, N, K, ab, cd):
    check_packed(dev, orc, M, N, K, ab, cd)


@pytest.mark.parametrize("M,N,K", [(768, 6144, 2048), (768, 8192, 2048), (768, 2048, 8192),
                                   (729, 3456, 1152), (729, 1152, 1152), (729, 4304, 1152), (729, 1152, 4304)])
@pytest.mark.parametrize("ab,cd", [(F16, F32), (BF16, F32), (BF16, BF16)])
def test_gemm_packed_model_shapes(dev, orc, M, N, K, ab, cd):
    """The Phi-1.5 prefill and SigLIP linears with fp16 and bf16 inputs (fp32 and
    bf16 out): every output column, 24 rows spread over M, within 1e-3 * S of the
    fp32 fma chain in ascending k (gemm.cl:26-51's arithmetic on 16-bit inputs)."""
    check_packed(dev, orc, M, N, K, ab, cd, rows=24)


@pytest.mark.parametrize("M,N,K", [(3, 5, 1), (17, 33, 7), (64, 70, 9), (100, 130, 588), (729, 1152, 588)])
@pytest.mark.parametrize("ab,cd", [(F16, F32), (BF16, BF16)])
def test_gemm_packed_any_k(dev, orc, M, N, K, ab, cd):
    """K not a multiple of 8 (gemm_image takes any K, gemm.cl:157-200): A's rows are
    not 16-byte aligned, so they are copied zero-padded into the workspace first;
    729x1152x588 is SigLIP's patch embedding (3x14x14 patch values per token)"""
    check_packed(dev, orc, M, N, K, ab, cd, rows=None if M < 200 else 40)


@pytest.mark.parametrize("batch,M,N,K,lda,ldb,sA,sB", [(3, 33, 40, 13, 15, 17, 33 * 15 + 1, 40 * 17 + 3),
                                                       (2, 65, 64, 72, 77, 72, 65 * 77, 64 * 72),
                                                       (4, 16, 24, 5, 5, 5, 80, 120)])
def test_gemm_batched_unaligned_rows(dev, orc, batch, M, N, K, lda, ldb, sA, sB):
    """batched NT products whose K, leading dimensions or batch strides leave rows
    off the 16-byte grid (both operands padded into the workspace)"""
    nA = (batch - 1) * sA + (M - 1) * lda + K
    nB = (batch - 1) * sB + (N - 1) * ldb + K
    A = orc.normal_f16(nA, 401)
    B = orc.normal_f16(nB, 402)
    dC = dev.alloc(batch * M * N * 4)
    dev.gemm_batched(dev.upload(A), dev.upload(B), dC, batch, M, N, K, lda, ldb, N, sA, sB, M * N)
    got = dC.download(np.float32).reshape(batch, M, N)
    for b in range(batch):
        a = np.stack([A[b * sA + r * lda: b * sA + r * lda + K] for r in range(M)])
        w = np.stack([B[b * sB + r * ldb: b * sB + r * ldb + K] for r in range(N)])
        ref = orc.gemm_nk("f16", a.copy(), w.copy(), M, N, K)
        _, Sc = orc.gemm_f64(orc.f16_to_f32(a).astype(np.float64), orc.f16_to_f32(w).astype(np.float64), M, N, K)
        ok, worst = within(got[b], ref, Sc, 1e-3)
        assert ok, (b, worst)


def test_gemm_packed_kn_layout_equals_nk(dev, orc):
    check_packed(dev, orc, 50, 72, 96, F16, F32, layout=m.LAYOUT_KN)


def test_gemm_batched_qk(dev, orc):
    """16 heads of 729 x 72 . 72 x 729, Q and K head-interleaved [729, 16, 72] (attention.cl:44)."""
    H, S, D = 16, 729, 72
    Q = orc.normal_f16(S * H * D, 181)
    Kt = orc.normal_f16(S * H * D, 182)
    dQ, dK, dC = dev.upload(Q), dev.upload(Kt), dev.alloc(H * S * S * 4)
    dev.gemm_batched(dQ, dK, dC, H, S, S, D, H * D, H * D, S, D, D, S * S)
    got = dC.download(np.float32).reshape(H, S, S)
    for h in (0, 7, 15):
        q = Q.reshape(S, H, D)[:, h, :].copy()
        k = Kt.reshape(S, H, D)[:, h, :].copy()
        ref = orc.gemm_nk("f16", q, k, S, S, D)
        _, Sc = orc.gemm_f64(orc.f16_to_f32(q).astype(np.float64), orc.f16_to_f32(k).astype(np.float64), S, S, D)
        ok, worst = within(got[h], ref, Sc, 1e-3)
        assert ok, (h, worst)


# ---------------------------------------------------------------------------
# buffers, pool, events, host-side errors with a live device
# ---------------------------------------------------------------------------

def test_buffers_views_and_pool(dev):
    import ctypes
    from mvlm_amd import native
    b = dev.alloc(1024)
    b.upload(np.arange(256, dtype=np.float32))
    v = b.view(512, 256)
    assert np.array_equal(v.download(np.float32), np.arange(128, 192, dtype=np.float32))
    with pytest.raises(native.MvlmError) as e:
        b.free()                       # a live view keeps the parent
    assert e.value.code == native.ERR_INVALID_ARG
    v.free()
    b.zero()
    dev.sync()
    assert not b.download(np.float32).any()
    L = native.lib()
    pool = ctypes.c_void_p()
    native.check(L.mvlm_pool_init(dev.handle, 4096, ctypes.byref(pool)), "pool_init")
    cur, nxt = L.mvlm_pool_current(pool), L.mvlm_pool_next(pool)
    assert cur and nxt and cur != nxt
    native.check(L.mvlm_pool_swap(pool), "swap")
    assert L.mvlm_pool_current(pool) == nxt and L.mvlm_pool_next(pool) == cur
    assert L.mvlm_buffer_size(cur) == 4096
    native.check(L.mvlm_pool_destroy(pool), "destroy")


def test_errors_with_live_device(dev):
    from mvlm_amd import native
    A, B, C = dev.alloc(64), dev.alloc(64), dev.alloc(8)
    with pytest.raises(native.MvlmError) as e:
        dev.gemm_naive(A, B, C, 4, 4, 4)           # C needs 32 bytes
    assert e.value.code == native.ERR_BUFFER_TOO_SMALL
    with pytest.raises(native.MvlmError) as e:
        dev.gemm_naive(A, B, C, 0, 4, 4)
    assert e.value.code == native.ERR_INVALID_ARG
    with pytest.raises(native.MvlmError) as e:
        dev.pack(np.zeros(18 * 2, np.uint8), Q4, 2, 30)   # K not a multiple of 32
    assert e.value.code == native.ERR_INVALID_ARG
    W = dev.pack(np.zeros(34 * 2, np.uint8), Q8, 1, 64)
    x, y = dev.alloc(64 * 4 * 17), dev.alloc(4 * 17)
    with pytest.raises(native.MvlmError) as e:
        dev.gemm_q8_0(x, W, y, 17, 1, 64)          # M above 16
    assert e.value.code == native.ERR_INVALID_ARG
    with pytest.raises(native.MvlmError) as e:
        dev.gemv_q4_0(x, W, y, 1, 64)              # wrong weight type
    assert e.value.code == native.ERR_INVALID_ARG
    Wf = dev.pack(np.zeros(3 * 12, np.uint16), F16, 3, 12)
    with pytest.raises(native.MvlmError) as e:
        dev.gemm_packed(dev.alloc(12 * 2 * 2 - 2), F16, Wf, dev.alloc(64), F32, 2, 3, 12)   # A one element short
    assert e.value.code == native.ERR_BUFFER_TOO_SMALL


def test_event_timing(dev, orc):
    N, K = 8192, 2048
    W = dev.random_weight(Q8, N, K, 5)
    x, y = dev.alloc(K * 4), dev.alloc(N * 4)
    dev.fill_normal(x, F32, K, 6)
    ev = dev.gemv_q8_0(x, W, y, N, K, event=True)
    ev.wait()
    ms = ev.elapsed_ms()
    assert 0.0 < ms < 100.0
    m0 = dev.marker()
    dev.gemv_q8_0(x, W, y, N, K)
    m1 = dev.marker()
    from mvlm_amd import native
    import ctypes
    t = ctypes.c_float()
    native.check(native.lib().mvlm_marker_elapsed_ms(m0.handle, m1.handle, ctypes.byref(t)), "marker")
    assert t.value > 0.0


# ---------------------------------------------------------------------------
# grouped decode GEMV (independent projections of one Phi-1.5 block, one launch)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("qt", [Q8, Q4])
def test_gemv_grouped_phi_block(dev, orc, qt):
    """QKV + fc1 share the block input; dense + fc2 read the attention / MLP branches."""
    shapes = [(6144, 2048, 0), (8192, 2048, 0), (2048, 2048, 1), (2048, 8192, 2)]
    xs_host = [orc.normal_f32(2048, 191), orc.normal_f32(2048, 192), orc.normal_f32(8192, 193)]
    xs = [dev.upload(v) for v in xs_host]
    blocks = [make_quant(orc, qt, N, K, 194 + i) for i, (N, K, _) in enumerate(shapes)]
    Ws = [dev.pack(b, qt, N, K) for b, (N, K, _) in zip(blocks, shapes)]
    ys = [dev.alloc(N * 4) for N, _, _ in shapes]
    ys1 = [dev.alloc(N * 4) for N, _, _ in shapes]
    dev.gemv_grouped([(xs[xi], F32, W, y, F32) for (N, K, xi), W, y in zip(shapes[:2], Ws[:2], ys[:2])])
    dev.gemv_grouped([(xs[xi], F32, W, y, F32) for (N, K, xi), W, y in zip(shapes[2:], Ws[2:], ys[2:])])
    kind = "q8_0" if qt == Q8 else "q4_0"
    deq = orc.dequant_q8_0 if qt == Q8 else orc.dequant_q4_0
    for (N, K, xi), W, b, y, y1 in zip(shapes, Ws, blocks, ys, ys1):
        dev.gemv(xs[xi], F32, W, y1, F32, N, K)
        got = y.download(np.float32)
        assert np.array_equal(got, y1.download(np.float32))      # same kernel, same bits
        ref = orc.gemm_nk(kind, xs_host[xi], b, 1, N, K)[0]
        _, S = orc.gemm_f64(xs_host[xi].astype(np.float64)[None], deq(b).astype(np.float64).reshape(N, K), 1, N, K)
        ok, worst = within(got, ref, S[0], 1e-5)
        assert ok, (N, K, worst)


@pytest.mark.parametrize("qt", [Q8, Q4])
def test_gemv_grouped_few_rows(dev, orc, qt):
    """2 KiB rows (Q8_0 K=2048, Q4_0 K=4096) and few rows: one row per wave,
    grouped with a problem of another work shape"""
    K2 = 2048 if qt == Q8 else 4096
    shapes = [(2048, K2), (300, K2 - 1024), (512, 1024)]
    kind = "q8_0" if qt == Q8 else "q4_0"
    deq = orc.dequant_q8_0 if qt == Q8 else orc.dequant_q4_0
    xh = [orc.normal_f32(K, 301 + i) for i, (_, K) in enumerate(shapes)]
    blocks = [make_quant(orc, qt, N, K, 311 + i) for i, (N, K) in enumerate(shapes)]
    Ws = [dev.pack(b, qt, N, K) for b, (N, K) in zip(blocks, shapes)]
    xs = [dev.upload(v) for v in xh]
    ys = [dev.alloc(N * 4) for N, _ in shapes]
    dev.gemv_grouped([(x, F32, W, y, F32) for x, W, y in zip(xs, Ws, ys)])
    for (N, K), x, b, y in zip(shapes, xh, blocks, ys):
        ref = orc.gemm_nk(kind, x, b, 1, N, K)[0]
        _, S = orc.gemm_f64(x.astype(np.float64)[None], deq(b).astype(np.float64).reshape(N, K), 1, N, K)
        ok, worst = within(y.download(np.float32), ref, S[0], 1e-5)
        assert ok, (N, K, worst)


def test_quant_rows_beyond_every_kernel_are_refused(dev):
    """Q8_0 rows of 131072 weights: too long for the streaming kernel (16 KiB) and
    their block scales overflow the skinny kernel's LDS: refused when the op is
    made, before anything is enqueued or captured"""
    from mvlm_amd import native
    N, K = 2, 131072
    W = dev.pack(np.zeros(34 * N * K // 32, np.uint8), Q8, N, K)
    x, y = dev.alloc(16 * K * 4), dev.alloc(16 * N * 4)
    for M in (1, 8):
        with pytest.raises(native.MvlmError) as e:
            dev.gemm_q8_0(x, W, y, M, N, K)
        assert e.value.code == native.ERR_UNSUPPORTED, M
        plan = m.Plan(dev)
        with pytest.raises(native.MvlmError) as e:
            plan.add_gemv(x, F32, W, y, F32, M)
        assert e.value.code == native.ERR_UNSUPPORTED, M
        plan.destroy()
    with pytest.raises(native.MvlmError) as e:
        dev.gemm_quant_grouped(8, [(x, F32, W, y, F32)])
    assert e.value.code == native.ERR_UNSUPPORTED


@pytest.mark.parametrize("qt", [Q8, Q4])
@pytest.mark.parametrize("M", [2, 4, 5, 16])
def test_gemm_quant_grouped(dev, orc, qt, M):
    """M rows of activations through a grouped launch (two groups shaped like a
    Phi-1.5 block's, smaller N): M <= 4 runs the streaming kernel (same bits as
    the single-op launches), M > 4 the matrix-core skinny kernel"""
    shapes = [(1536, 2048, 0), (2048, 2048, 0), (512, 2048, 1), (512, 8192, 2)]
    xs_host = [orc.normal_f32(M * 2048, 261), orc.normal_f32(M * 2048, 262), orc.normal_f32(M * 8192, 263)]
    xs = [dev.upload(v) for v in xs_host]
    blocks = [make_quant(orc, qt, N, K, 264 + i) for i, (N, K, _) in enumerate(shapes)]
    Ws = [dev.pack(b, qt, N, K) for b, (N, K, _) in zip(blocks, shapes)]
    ys = [dev.alloc(M * N * 4) for N, _, _ in shapes]
    dev.gemm_quant_grouped(M, [(xs[xi], F32, W, y, F32) for (N, K, xi), W, y in zip(shapes[:2], Ws[:2], ys[:2])])
    plan = m.Plan(dev)
    plan.add_gemm_quant_grouped(M, [(xs[xi], F32, W, y, F32) for (N, K, xi), W, y in zip(shapes[2:], Ws[2:], ys[2:])])
    plan.use_graph(True)
    plan.run(2)
    dev.sync()
    kind = "q8_0" if qt == Q8 else "q4_0"
    deq = orc.dequant_q8_0 if qt == Q8 else orc.dequant_q4_0
    single = dev.gemm_q8_0 if qt == Q8 else dev.gemm_q4_0
    for (N, K, xi), W, b, y in zip(shapes, Ws, blocks, ys):
        got = y.download(np.float32).reshape(M, N)
        if M <= 4:
            y1 = dev.alloc(M * N * 4)
            single(xs[xi], W, y1, M, N, K)
            assert np.array_equal(got, y1.download(np.float32).reshape(M, N))
        X = xs_host[xi].reshape(M, K)
        ref = orc.gemm_nk(kind, X.ravel(), b, M, N, K)
        _, S = orc.gemm_f64(X.astype(np.float64), deq(b).astype(np.float64).reshape(N, K), M, N, K)
        ok, worst = within(got, ref.reshape(M, N), S.reshape(M, N), 1e-5)
        assert ok, (M, N, K, worst)


@pytest.mark.parametrize("qt", [Q8, Q4])
@pytest.mark.parametrize("M", [9, 16])
def test_gemm_quant_grouped_phi_qkv_fc1(dev, orc, qt, M):
    """the QKV + fc1 group of a Phi-1.5 block at full size (6144 + 8192 rows
    over one x, 896 row groups): the skinny kernel's four-row-group shape"""
    shapes = [(6144, 2048), (8192, 2048)]
    kind = "q8_0" if qt == Q8 else "q4_0"
    deq = orc.dequant_q8_0 if qt == Q8 else orc.dequant_q4_0
    xh = orc.normal_f32(M * 2048, 301)
    x = dev.upload(xh)
    blocks = [make_quant(orc, qt, N, K, 302 + i) for i, (N, K) in enumerate(shapes)]
    Ws = [dev.pack(b, qt, N, K) for b, (N, K) in zip(blocks, shapes)]
    Ys = [dev.alloc(M * N * 4) for N, _ in shapes]
    dev.gemm_quant_grouped(M, [(x, F32, W, y, F32) for W, y in zip(Ws, Ys)])
    for (N, K), b, y in zip(shapes, blocks, Ys):
        ref = orc.gemm_nk(kind, xh, b, M, N, K)
        _, S = orc.gemm_f64(xh.astype(np.float64).reshape(M, K), deq(b).astype(np.float64).reshape(N, K), M, N, K)
        ok, worst = within(y.download(np.float32).reshape(M, N), ref.reshape(M, N), S.reshape(M, N), 1e-5)
        assert ok, (M, N, K, worst)


@pytest.mark.parametrize("qt", [Q8, Q4])
@pytest.mark.parametrize("M", [3, 7])
def test_gemm_quant_grouped_ragged(dev, orc, qt, M):
    """ragged row counts (not multiples of the 16-row tile or of the block's
    rows) and different K in one group: blocks are dealt to the problems in
    order and each block stages its own problem's K"""
    shapes = [(17, 96), (300, 2048), (33, 1024), (1, 32), (129, 8192)]
    kind = "q8_0" if qt == Q8 else "q4_0"
    deq = orc.dequant_q8_0 if qt == Q8 else orc.dequant_q4_0
    Xh = [orc.normal_f32(M * K, 281 + i) for i, (_, K) in enumerate(shapes)]
    blocks = [make_quant(orc, qt, N, K, 291 + i) for i, (N, K) in enumerate(shapes)]
    Ws = [dev.pack(b, qt, N, K) for b, (N, K) in zip(blocks, shapes)]
    Xs = [dev.upload(x) for x in Xh]
    Ys = [dev.alloc(M * N * 4) for N, _ in shapes]
    dev.gemm_quant_grouped(M, [(x, F32, W, y, F32) for x, W, y in zip(Xs, Ws, Ys)])
    for (N, K), x, b, y in zip(shapes, Xh, blocks, Ys):
        ref = orc.gemm_nk(kind, x, b, M, N, K)
        _, S = orc.gemm_f64(x.astype(np.float64).reshape(M, K), deq(b).astype(np.float64).reshape(N, K), M, N, K)
        ok, worst = within(y.download(np.float32).reshape(M, N), ref.reshape(M, N), S.reshape(M, N), 1e-5)
        assert ok, (M, N, K, worst)


def test_gemm_quant_grouped_errors(dev):
    from mvlm_amd import native
    x, y = dev.alloc(4 * 65536), dev.alloc(4 * 65536)
    W8 = dev.pack(np.zeros(34 * 64, np.uint8), Q8, 64, 1024)
    W4 = dev.pack(np.zeros(18 * 64, np.uint8), Q4, 64, 1024)
    Wh = dev.pack(np.zeros(64 * 1024, np.uint16), F16, 64, 1024)
    for M, entries, code in ((4, [(x, F32, W8, y, F32), (x, F32, W4, y, F32)], native.ERR_INVALID_ARG),
                             (0, [(x, F32, W8, y, F32)], native.ERR_INVALID_ARG),
                             (17, [(x, F32, W8, y, F32)], native.ERR_INVALID_ARG),
                             (2, [(x, F16, Wh, y, F32)], native.ERR_INVALID_ARG),       # dense weights
                             (1, [(x, F16, Wh, y, F32)], native.ERR_INVALID_ARG),       # also at M == 1
                             (8, [(x, F16, W8, y, F32)], native.ERR_INVALID_ARG)):      # fp32 x for quant
        with pytest.raises(native.MvlmError) as e:
            dev.gemm_quant_grouped(M, entries)
        assert e.value.code == code, (M, e.value)


def test_gemv_grouped_dense_and_plan(dev, orc):
    shapes = [(300, 512), (77, 1024), (1, 64)]
    xs_host = [orc.normal_f16(K, 201 + i) for i, (_, K) in enumerate(shapes)]
    Wh = [orc.normal_f16(N * K, 211 + i, 0.02) for i, (N, K) in enumerate(shapes)]
    xs = [dev.upload(v) for v in xs_host]
    Ws = [dev.pack(w, F16, N, K) for w, (N, K) in zip(Wh, shapes)]
    ys = [dev.alloc(N * 4) for N, _ in shapes]
    plan = m.Plan(dev)
    plan.add_gemv_grouped([(x, F16, W, y, F32) for x, W, y in zip(xs, Ws, ys)])
    plan.use_graph(True)
    plan.run(3)
    dev.sync()
    for (N, K), xh, wh, y in zip(shapes, xs_host, Wh, ys):
        ref, S = orc.gemm_f64(orc.f16_to_f32(xh).astype(np.float64)[None],
                              orc.f16_to_f32(wh).astype(np.float64).reshape(N, K), 1, N, K)
        ok, worst = within(y.download(np.float32), ref[0], S[0], 1e-3)
        assert ok, worst


def test_gemv_grouped_errors(dev):
    from mvlm_amd import native
    x, y = dev.alloc(4 * 65536), dev.alloc(4 * 4096)
    W8 = dev.pack(np.zeros(34 * 64, np.uint8), Q8, 64, 1024)
    W4 = dev.pack(np.zeros(18 * 64, np.uint8), Q4, 64, 1024)
    with pytest.raises(native.MvlmError) as e:           # mixed weight formats
        dev.gemv_grouped([(x, F32, W8, y, F32), (x, F32, W4, y, F32)])
    assert e.value.code == native.ERR_INVALID_ARG
    with pytest.raises(native.MvlmError) as e:           # more than MVLM_MAX_GROUP entries
        dev.gemv_grouped([(x, F32, W8, y, F32)] * 9)
    assert e.value.code == native.ERR_INVALID_ARG
    Wlong = dev.pack(np.zeros(34 * 2048, np.uint8), Q8, 1, 65536)   # 64 KiB rows
    with pytest.raises(native.MvlmError) as e:
        dev.gemv_grouped([(x, F32, Wlong, y, F32)])
    assert e.value.code == native.ERR_UNSUPPORTED
    dev.gemv(x, F32, Wlong, y, F32, 1, 65536)            # the single entry point still serves it


@pytest.mark.parametrize("splits", ["2", "3", "4"])
@pytest.mark.parametrize("M,N,K,ab,cd", [(129, 130, 1000, F16, BF16), (768, 256, 2048, F16, F32),
                                         (33, 65, 1032, BF16, F16)])
def test_gemm_forced_k_splits(dev, orc, monkeypatch, splits, M, N, K, ab, cd):
    """K split over workgroups (fp32 partials in the device workspace, summed in
    split order by a second kernel), including a K tail past the last full stage"""
    monkeypatch.setenv("MVLM_GEMM_SPLITS", splits)
    check_packed(dev, orc, M, N, K, ab, cd, seed=300 + int(splits))


@pytest.mark.parametrize("tile", ["256x256s2w8", "256x128s2w8", "192x128s3w8", "128x128s4w8", "64x64s4w4",
                                  "128x128s2w8k128", "64x64s2w4k128", "192x128s2w8k128", "96x192s2w6k128"])
@pytest.mark.parametrize("M,N,K,ab,cd", [(300, 410, 1000, F16, F32), (97, 200, 264, BF16, BF16)])
def test_gemm_every_automatic_tile(dev, orc, monkeypatch, tile, M, N, K, ab, cd):
    """each tile the planner can choose, forced, on shapes that leave partial
    tiles along M and N and a K tail past the last full stage"""
    monkeypatch.setenv("MVLM_GEMM_TILE", tile)
    check_packed(dev, orc, M, N, K, ab, cd, seed=320)


def test_gemm_k_splits_with_epilogue_and_batches(dev, orc, monkeypatch):
    from test_gpu_epilogue import check as ep_check, make_operands
    from mvlm_amd import native
    monkeypatch.setenv("MVLM_GEMM_SPLITS", "3")
    M, N, K = 96, 200, 1536
    A = orc.normal_f16(M * K, 0x310)
    Wt = orc.normal_f16(N * K, 0x311, 0.05)
    W = dev.pack(Wt, F16, N, K)
    ops, vals = make_operands(dev, orc, M, N, F32, 0x312, True, True, True)
    C = ops["residual"]                                    # in-place residual add
    dev.gemm_packed_ex(dev.upload(A), F16, W, C, F32, M, N, K, bias=ops["bias"], act=native.ACT_GELU_TANH,
                       mul=ops["mul"], residual=C)
    got = C.download(np.float32, M * N).astype(np.float64).reshape(M, N)
    Y64, S = orc.gemm_f64(widen(orc, A, F16).reshape(M, K), widen(orc, Wt, F16).reshape(N, K), M, N, K)
    ep_check(orc, got, Y64, S, vals, native.ACT_GELU_TANH, F32, 1e-4)
    # batched Q K^T with splits: every head equals its own unsplit product within tolerance
    H, Sq, D = 4, 100, 512
    Q = orc.normal_f16(Sq * H * D, 0x313)
    Kt = orc.normal_f16(Sq * H * D, 0x314)
    dQ, dK, dC = dev.upload(Q), dev.upload(Kt), dev.alloc(H * Sq * Sq * 4)
    dev.gemm_batched(dQ, dK, dC, H, Sq, Sq, D, H * D, H * D, Sq, D, D, Sq * Sq)
    got = dC.download(np.float32).reshape(H, Sq, Sq)
    for h in range(H):
        q = Q.reshape(Sq, H, D)[:, h, :].copy()
        k = Kt.reshape(Sq, H, D)[:, h, :].copy()
        ref = orc.gemm_nk("f16", q, k, Sq, Sq, D)
        _, Sc = orc.gemm_f64(orc.f16_to_f32(q).astype(np.float64), orc.f16_to_f32(k).astype(np.float64), Sq, Sq, D)
        ok, worst = within(got[h], ref, Sc, 1e-3)
        assert ok, (h, worst)
