"""ctypes binding of oracle/liboracle.so — TEST INFRASTRUCTURE.

The oracle is the checker: the test suite, the smoke check and the benchmark's
CPU-baseline leg load it; the product library never does.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")

_lib = None


def build() -> None:
    """Compile liboracle.so with the committed Makefile (gcc, no GPU needed)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        sz, i, u64, d = ctypes.c_size_t, ctypes.c_int, ctypes.c_uint64, ctypes.c_double
        sig = {
            "orc_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
            "orc_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "orc_f32_to_bf16": (ctypes.c_uint16, [ctypes.c_float]),
            "orc_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "orc_f32_to_f16_array": (None, [_f32p, _u16p, sz]),
            "orc_f16_to_f32_array": (None, [_u16p, _f32p, sz]),
            "orc_f32_to_bf16_array": (None, [_f32p, _u16p, sz]),
            "orc_bf16_to_f32_array": (None, [_u16p, _f32p, sz]),
            "orc_splitmix64_at": (u64, [u64, u64]),
            "orc_uniform_at": (d, [u64, u64]),
            "orc_normal_at": (d, [u64, u64]),
            "orc_fill_normal_f32": (None, [_f32p, sz, u64, d]),
            "orc_fill_normal_f16": (None, [_u16p, sz, u64, d]),
            "orc_fill_normal_bf16": (None, [_u16p, sz, u64, d]),
            "orc_fill_q8_0": (None, [_u8p, sz, u64, d]),
            "orc_fill_q4_0": (None, [_u8p, sz, u64, d]),
            "orc_ggml_type_size": (i, [i]),
            "orc_ggml_block_size": (i, [i]),
            "orc_dequant_q8_0": (None, [_u8p, _f32p, sz]),
            "orc_dequant_q4_0": (None, [_u8p, _f32p, sz]),
            "orc_gemm_naive": (None, [_u16p, _u16p, _u16p, _f32p, i, i, i]),
            "orc_gemm_tiled": (None, [_u16p, _u16p, _u16p, _f32p, i, i, i]),
            "orc_gemm_image": (None, [_u16p, _u16p, _u16p, _f32p, i, i, i]),
            "orc_gemv": (None, [_u16p, _u16p, _u16p, _f32p, i, i]),
            "orc_gemm_image_mt": (None, [_u16p, _u16p, _u16p, _f32p, i, i, i, i]),
            "orc_gemv_mt": (None, [_u16p, _u16p, _u16p, _f32p, i, i, i]),
            "orc_gemm_f32_nk": (None, [_f32p, _f32p, _f32p, i, i, i, i]),
            "orc_gemm_f16_nk": (None, [_u16p, _u16p, _f32p, i, i, i, i]),
            "orc_gemm_bf16_nk": (None, [_u16p, _u16p, _f32p, i, i, i, i]),
            "orc_gemm_q8_0_nk": (None, [_f32p, _u8p, _f32p, i, i, i, i]),
            "orc_gemm_q4_0_nk": (None, [_f32p, _u8p, _f32p, i, i, i, i]),
            "orc_gemm_batched_f16": (None, [_u16p, _u16p, _f32p, i, i, i, i,
                                            ctypes.c_long, ctypes.c_long, ctypes.c_long,
                                            ctypes.c_long, ctypes.c_long, ctypes.c_long]),
            "orc_gemm_f64_nk": (None, [_f64p, _f64p, _f64p, _f64p, i, i, i, i]),
            "orc_max_threads": (i, []),
            "orc_argmax_f16_reference": (i, [_u16p, i]),
            "orc_argmax": (None, [ctypes.c_void_p, i, i, i, ctypes.c_long, np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")]),
            "orc_attention_f64": (None, [_u16p, _u16p, _u16p, _f64p, _f64p, _f64p, i, i, i, i, i, d, i]),
            "orc_gelu_tanh": (d, [d]),
            "orc_silu": (d, [d]),
            "orc_epilogue_f64": (None, [_f64p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, i, i, i]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


# ---- convenience wrappers (numpy in, numpy out) ---------------------------

SEED_BASE = 0x4D564C4D


def seed_for(tensor_id: int) -> int:
    return SEED_BASE ^ tensor_id


def normal_f32(n, seed, std=1.0):
    out = np.empty(n, np.float32)
    lib().orc_fill_normal_f32(out, n, seed, std)
    return out


def normal_f16(n, seed, std=1.0):
    out = np.empty(n, np.uint16)
    lib().orc_fill_normal_f16(out, n, seed, std)
    return out


def normal_bf16(n, seed, std=1.0):
    out = np.empty(n, np.uint16)
    lib().orc_fill_normal_bf16(out, n, seed, std)
    return out


def q8_0_blocks(nblocks, seed, wstd=0.02):
    out = np.empty(nblocks * 34, np.uint8)
    lib().orc_fill_q8_0(out, nblocks, seed, wstd)
    return out


def q4_0_blocks(nblocks, seed, wstd=0.02):
    out = np.empty(nblocks * 18, np.uint8)
    lib().orc_fill_q4_0(out, nblocks, seed, wstd)
    return out


def f16_to_f32(h):
    h = np.ascontiguousarray(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_f16_to_f32_array(h.ravel(), out.ravel(), h.size)
    return out


def f32_to_f16(f):
    f = np.ascontiguousarray(f, np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().orc_f32_to_f16_array(f.ravel(), out.ravel(), f.size)
    return out


def bf16_to_f32(h):
    h = np.ascontiguousarray(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_bf16_to_f32_array(h.ravel(), out.ravel(), h.size)
    return out


def f32_to_bf16(f):
    f = np.ascontiguousarray(f, np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().orc_f32_to_bf16_array(f.ravel(), out.ravel(), f.size)
    return out


def dequant_q8_0(blocks):
    nb = blocks.size // 34
    out = np.empty(nb * 32, np.float32)
    lib().orc_dequant_q8_0(np.ascontiguousarray(blocks, np.uint8), out, nb)
    return out


def dequant_q4_0(blocks):
    nb = blocks.size // 18
    out = np.empty(nb * 32, np.float32)
    lib().orc_dequant_q4_0(np.ascontiguousarray(blocks, np.uint8), out, nb)
    return out


def _ref_kn(fn, A, B, M, N, K):
    C16 = np.empty(M * N, np.uint16)
    C32 = np.empty(M * N, np.float32)
    fn(np.ascontiguousarray(A, np.uint16).ravel(), np.ascontiguousarray(B, np.uint16).ravel(),
       C16, C32, M, N, K)
    return C16.reshape(M, N), C32.reshape(M, N)


def gemm_naive(A, B, M, N, K):
    return _ref_kn(lib().orc_gemm_naive, A, B, M, N, K)


def gemm_tiled(A, B, M, N, K):
    return _ref_kn(lib().orc_gemm_tiled, A, B, M, N, K)


def gemm_image(A, B, M, N, K):
    return _ref_kn(lib().orc_gemm_image, A, B, M, N, K)


def gemv(x, B, N, K, nthreads=1):
    y16 = np.empty(N, np.uint16)
    y32 = np.empty(N, np.float32)
    lib().orc_gemv_mt(np.ascontiguousarray(x, np.uint16).ravel(), np.ascontiguousarray(B, np.uint16).ravel(),
                      y16, y32, N, K, nthreads)
    return y16, y32


def gemm_image_mt(A, B, M, N, K, nthreads=0):
    C16 = np.empty(M * N, np.uint16)
    C32 = np.empty(M * N, np.float32)
    lib().orc_gemm_image_mt(np.ascontiguousarray(A, np.uint16).ravel(), np.ascontiguousarray(B, np.uint16).ravel(),
                            C16, C32, M, N, K, nthreads)
    return C16.reshape(M, N), C32.reshape(M, N)


def gemm_nk(kind, X, W, M, N, K, nthreads=0):
    Y = np.empty(M * N, np.float32)
    fn = {"f32": lib().orc_gemm_f32_nk, "f16": lib().orc_gemm_f16_nk, "bf16": lib().orc_gemm_bf16_nk,
          "q8_0": lib().orc_gemm_q8_0_nk, "q4_0": lib().orc_gemm_q4_0_nk}[kind]
    xdt = np.float32 if kind in ("f32", "q8_0", "q4_0") else np.uint16
    wdt = {"f32": np.float32, "f16": np.uint16, "bf16": np.uint16, "q8_0": np.uint8, "q4_0": np.uint8}[kind]
    fn(np.ascontiguousarray(X, xdt).ravel(), np.ascontiguousarray(W, wdt).ravel(), Y, M, N, K, nthreads)
    return Y.reshape(M, N)


def gemm_f64(X, W, M, N, K, nthreads=0):
    """fp64 brute force of X[M,K] * W[N,K]^T and the scale sum_k |x*w|."""
    Y = np.empty(M * N, np.float64)
    S = np.empty(M * N, np.float64)
    lib().orc_gemm_f64_nk(np.ascontiguousarray(X, np.float64).ravel(),
                          np.ascontiguousarray(W, np.float64).ravel(), Y, S, M, N, K, nthreads)
    return Y.reshape(M, N), S.reshape(M, N)


def epilogue_f64(Y, bias=None, mul=None, res=None, act=0):
    """Y[M,N] (fp64, updated copy) -> act(Y + bias[n]) * mul + res."""
    Y = np.array(Y, np.float64, copy=True)
    M, N = Y.shape

    def ptr(a, n):
        if a is None:
            return None
        a = np.ascontiguousarray(a, np.float64).ravel()
        assert a.size == n
        keep.append(a)
        return a.ctypes.data
    keep = []
    lib().orc_epilogue_f64(Y.ravel(), ptr(bias, N), ptr(mul, M * N), ptr(res, M * N), act, M, N)
    return Y


def gemm_batched_f16(A, B, batch, M, N, K, lda, ldb, ldc, sA, sB, sC, c_elems):
    C = np.zeros(c_elems, np.float32)
    lib().orc_gemm_batched_f16(np.ascontiguousarray(A, np.uint16).ravel(),
                               np.ascontiguousarray(B, np.uint16).ravel(), C,
                               batch, M, N, K, lda, ldb, ldc, sA, sB, sC)
    return C


def attention_f64(Q, K, V, seq_q, seq_kv, heads, D, causal=False, scale=None, nthreads=0):
    """fp64 attention of fp16-bit Q/K/V ([seq][heads][D]); returns (O, A, R):
    O and A = sum_k p_k |V_k| as [seq_q, heads, D], R = max_k scale sum_d |q k| as [seq_q, heads]."""
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    O = np.empty(seq_q * heads * D, np.float64)
    A = np.empty_like(O)
    R = np.empty(seq_q * heads, np.float64)
    lib().orc_attention_f64(np.ascontiguousarray(Q, np.uint16).ravel(), np.ascontiguousarray(K, np.uint16).ravel(),
                            np.ascontiguousarray(V, np.uint16).ravel(), O, A, R, seq_q, seq_kv, heads, D,
                            1 if causal else 0, float(scale), nthreads)
    return O.reshape(seq_q, heads, D), A.reshape(seq_q, heads, D), R.reshape(seq_q, heads)


def argmax(x, dtype, rows, n, ld):
    """row-wise first index of the largest key (x: float32 array or uint16 bits)."""
    x = np.ascontiguousarray(x)
    out = np.empty(rows, np.int32)
    lib().orc_argmax(x.ctypes.data, dtype, rows, n, ld, out)
    return out
