"""mvlm_gemm_packed_ex_noalloc: the packed GEMM with its workspace (K-split
partials, the zero-padded copy of A when K % 8 != 0) in the library's fixed
per-GPU array instead of an allocation.  Its output must equal
mvlm_gemm_packed_ex's bit for bit (same kernels, same split order), on calls
in a row whose second one is smaller, and a shape needing more than the fixed
array is refused on the host."""
from __future__ import annotations

import numpy as np
import pytest

import mvlm_amd as m
from mvlm_amd import native

pytestmark = pytest.mark.gpu

F16, F32 = m.F16, m.F32
NOALLOC_BYTES = 32 << 20


def operands(dev, orc, M, N, K, cd, seed):
    """A, W and a bias of the output's dtype (the epilogue's operands share it)"""
    A = dev.upload(orc.normal_f16(M * K, seed))
    W = dev.pack(orc.normal_f16(N * K, seed + 1, 0.02), F16, N, K)
    bias = dev.upload(orc.normal_f32(N, seed + 2) if cd == F32 else orc.normal_f16(N, seed + 2))
    return A, W, bias


def poisoned(dev, nbytes):
    """an output buffer holding NaN patterns, so an element left unwritten shows"""
    return dev.upload(np.full(nbytes // 2, 0x7E00, np.uint16))


def run_both(dev, orc, M, N, K, cd, seed):
    A, W, bias = operands(dev, orc, M, N, K, cd, seed)
    es = 4 if cd == F32 else 2
    c_ref, c_new = poisoned(dev, M * N * es), poisoned(dev, M * N * es)
    dev.gemm_packed_ex(A, F16, W, c_ref, cd, M, N, K, bias=bias)
    dev.gemm_packed_ex_noalloc(A, F16, W, c_new, cd, M, N, K, bias=bias)
    dev.sync()
    got, ref = c_new.download(np.uint8), c_ref.download(np.uint8)
    assert np.array_equal(got, ref), (M, N, K)
    vals = got.view(np.float32 if cd == F32 else np.float16)
    assert np.all(np.isfinite(vals)), (M, N, K)


@pytest.mark.parametrize("order", ["large_then_small", "small_then_large"])
def test_noalloc_matches_allocating_entry(dev, orc, monkeypatch, order):
    # Phi-1.5 fc2 at 768 tokens takes a 4-way K split (25 MB of partials);
    # 129x130x1000 with a forced 3-way split and 100x130x588 (A padded to
    # K=592) leave different contents of the shared array behind
    cases = [(768, 2048, 8192, F32, None), (129, 130, 1000, F16, "3"), (100, 130, 588, F32, None)]
    if order == "small_then_large":
        cases = cases[::-1]
    for i, (M, N, K, cd, splits) in enumerate(cases):
        if splits:
            monkeypatch.setenv("MVLM_GEMM_SPLITS", splits)
        else:
            monkeypatch.delenv("MVLM_GEMM_SPLITS", raising=False)
        print(f"[noalloc] {order} call {i}: {M}x{N}x{K} splits={splits}", flush=True)
        run_both(dev, orc, M, N, K, cd, 0x900 + 16 * i)


def test_noalloc_refuses_workspace_beyond_the_array(dev, orc, monkeypatch):
    # an 8-way split of a 1024 x 2048 output: 64 MiB of partials
    monkeypatch.setenv("MVLM_GEMM_SPLITS", "8")
    M, N, K = 1024, 2048, 4096
    assert 8 * M * N * 4 > NOALLOC_BYTES
    A, W, _ = operands(dev, orc, M, N, K, F32, 0x950)
    C = dev.alloc(M * N * 4)
    with pytest.raises(native.MvlmError) as e:
        dev.gemm_packed_ex_noalloc(A, F16, W, C, F32, M, N, K)
    assert e.value.code == native.ERR_UNSUPPORTED
