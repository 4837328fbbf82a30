"""The small-K batched product (gemm_smallk.hip): NT products with K <= 128 and
a dense fp32 C, which each workgroup writes as one contiguous range of 16 rows
with 16-byte stores aligned in memory.  Checked on every element against the
oracle's fp32 fma chain (1e-3 * S, S = sum_k |a_k b_k|), over shapes whose
ranges start at every alignment modulo 16 bytes, row blocks cut short at M,
column counts that are not multiples of 16, K from 8 to 128, workgroups with
more A rows to stage than their threads load ahead of B (48 x 400 x 40 x 128),
and with the bytes between batches (sC > M N) and after C left untouched."""
from __future__ import annotations

import numpy as np
import pytest

import mvlm_amd as m
from conftest import within

pytestmark = pytest.mark.gpu

SENTINEL = np.float32(-7.25)


@pytest.mark.parametrize("batch,M,N,K,gap", [(1, 1, 1, 8, 0), (2, 15, 5, 24, 3), (3, 17, 33, 64, 1),
                                             (2, 16, 16, 128, 0), (3, 40, 129, 72, 5), (2, 33, 1023, 120, 2),
                                             (16, 729, 729, 72, 0), (48, 400, 40, 128, 1)])
def test_smallk_batched_every_element(dev, orc, batch, M, N, K, gap):
    print(f"[smallk] batch={batch} M={M} N={N} K={K} gap={gap}", flush=True)
    H = batch
    lda = ldb = H * K                       # head-interleaved rows, as Q and K of attention
    sA = sB = K
    sC = M * N + gap
    A = orc.normal_f16(M * lda, 500 + M)
    B = orc.normal_f16(N * ldb, 600 + N)
    total = batch * sC + 7
    dC = dev.upload(np.full(total, SENTINEL, np.float32))
    dev.gemm_batched(dev.upload(A), dev.upload(B), dC, batch, M, N, K, lda, ldb, N, sA, sB, sC)
    got = dC.download(np.float32)
    for b in range(batch):
        a = A.reshape(M, H, K)[:, b, :].copy()
        w = B.reshape(N, H, K)[:, b, :].copy()
        ref = orc.gemm_nk("f16", a, w, M, N, K)
        _, S = orc.gemm_f64(orc.f16_to_f32(a).astype(np.float64), orc.f16_to_f32(w).astype(np.float64), M, N, K)
        ok, worst = within(got[b * sC: b * sC + M * N].reshape(M, N), ref, S, 1e-3)
        assert ok, (b, worst)
        assert np.all(got[b * sC + M * N: (b + 1) * sC] == SENTINEL), b   # the gap between batches
    assert np.all(got[batch * sC:] == SENTINEL)


@pytest.mark.parametrize("M,N,K", [(5, 7, 16), (33, 65, 40), (129, 130, 120)])
def test_smallk_bf16_through_packed_weights(dev, orc, M, N, K):
    """bf16 A and packed bf16 W with K <= 128 take the same path"""
    A = orc.normal_bf16(M * K, 701)
    Wt = orc.normal_bf16(N * K, 702, 0.02)
    W = dev.pack(Wt, m.BF16, N, K)
    dC = dev.alloc(M * N * 4)
    dev.gemm_packed(dev.upload(A), m.BF16, W, dC, m.F32, M, N, K)
    got = dC.download(np.float32).reshape(M, N)
    ref = orc.gemm_nk("bf16", A, Wt, M, N, K)
    _, S = orc.gemm_f64(orc.bf16_to_f32(A).astype(np.float64).reshape(M, K),
                        orc.bf16_to_f32(Wt).astype(np.float64).reshape(N, K), M, N, K)
    ok, worst = within(got, ref, S, 1e-3)
    assert ok, worst


def test_smallk_unaligned_output_takes_the_general_path(dev, orc):
    """C 4 bytes past a 16-byte boundary: the general MFMA GEMM serves it, same results"""
    batch, M, N, K = 2, 20, 30, 72
    A = orc.normal_f16(batch * M * K, 801)
    B = orc.normal_f16(batch * N * K, 802)
    base = dev.alloc((batch * M * N + 4) * 4)
    dC = base.view(4, batch * M * N * 4)
    dev.gemm_batched(dev.upload(A), dev.upload(B), dC, batch, M, N, K, K, K, N, M * K, N * K, M * N)
    got = dC.download(np.float32).reshape(batch, M, N)
    for b in range(batch):
        a = A[b * M * K:(b + 1) * M * K].reshape(M, K)
        w = B[b * N * K:(b + 1) * N * K].reshape(N, K)
        ref = orc.gemm_nk("f16", a.copy(), w.copy(), M, N, K)
        _, S = orc.gemm_f64(orc.f16_to_f32(a).astype(np.float64), orc.f16_to_f32(w).astype(np.float64), M, N, K)
        ok, worst = within(got[b], ref, S, 1e-3)
        assert ok, (b, worst)
