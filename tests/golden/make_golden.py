"""Writes the golden fixtures under tests/golden/ (run: python tests/golden/make_golden.py).

Nothing here calls the oracle or the HIP library: every expected value comes
from the GGUF block definition evaluated with numpy's float16 decoding and
exact integer arithmetic, or from exact integer matrix products.

* blocks_known_answer.json — hand-built Q8_0 / Q4_0 blocks whose dequantized
  values are fixed by the GGUF definition (ggml block_q8_0 / block_q4_0, the
  34- and 18-byte blocks the reference pins in tests/test_gguf.cpp:16-34):
    Q8_0 w_j = d * qs_j
    Q4_0 w_j = ((qs_j & 15) - 8) * d,  w_{j+16} = ((qs_j >> 4) - 8) * d   (j < 16)
  The cases make the nibble order, the sign of int8 codes, subnormal and
  largest-finite fp16 scales observable.
* gemm_exact_int.npz — small-integer fp16 matrices whose products and every
  partial sum are exact in fp32 and fp16, so every summation order (naive,
  tiled, image, the 256-lane gemv tree, MFMA) must give these bits.
"""
from __future__ import annotations

import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def f16_bits(value: float) -> int:
    return int(np.array([value], np.float16).view(np.uint16)[0])


def f16_value(bits: int) -> float:
    return float(np.array([bits], np.uint16).view(np.float16)[0])


def q8_block(d_bits: int, qs: list[int]) -> dict:
    assert len(qs) == 32 and all(-128 <= q <= 127 for q in qs)
    raw = bytes([d_bits & 0xFF, d_bits >> 8]) + bytes((q & 0xFF) for q in qs)
    d = f16_value(d_bits)
    vals = [np.float32(q * d) for q in qs]          # exact: <= 19 significant bits
    assert all(float(v) == q * d for v, q in zip(vals, qs))
    return {"type": "q8_0", "bytes": raw.hex(), "values": [float(v) for v in vals],
            "bits": [int(np.array([v], np.float32).view(np.uint32)[0]) for v in vals]}


def q4_block(d_bits: int, codes: list[int]) -> dict:
    """codes[j] for weight j = 0..31 (each 0..15); byte j = codes[j] | codes[j+16] << 4."""
    assert len(codes) == 32 and all(0 <= c <= 15 for c in codes)
    qs = [codes[j] | (codes[j + 16] << 4) for j in range(16)]
    raw = bytes([d_bits & 0xFF, d_bits >> 8]) + bytes(qs)
    d = f16_value(d_bits)
    vals = [np.float32((c - 8) * d) for c in codes]
    assert all(float(v) == (c - 8) * d for v, c in zip(vals, codes))
    return {"type": "q4_0", "bytes": raw.hex(), "values": [float(v) for v in vals],
            "bits": [int(np.array([v], np.float32).view(np.uint32)[0]) for v in vals]}


def known_answer_blocks() -> list[dict]:
    one, half = f16_bits(1.0), f16_bits(0.5)
    cases = [
        ("q8 ramp -16..15, d=1", q8_block(one, list(range(-16, 16)))),
        ("q8 extremes, d=0.5", q8_block(half, [-127, 127, 0, 1, -1, 64, -64, 100] * 4)),
        ("q8 smallest subnormal d", q8_block(0x0001, [127, -127] * 16)),
        ("q8 largest finite d", q8_block(0x7BFF, [-127, 127, 3, -3] * 8)),
        ("q8 negative d", q8_block(f16_bits(-0.25), list(range(0, 32)))),
        ("q8 code -128", q8_block(one, [-128] + [0] * 31)),
        ("q4 nibble order, d=1", q4_block(one, list(range(16)) + [15 - j for j in range(16)])),
        ("q4 all codes, d=0.125", q4_block(f16_bits(0.125), [j % 16 for j in range(32)])),
        ("q4 zero point 8", q4_block(f16_bits(3.0), [8] * 32)),
        ("q4 subnormal d", q4_block(0x0003, [0, 15] * 16)),
        ("q4 largest finite d", q4_block(0x7BFF, [0, 15, 7, 9] * 8)),
    ]
    return [dict(name=n, **c) for n, c in cases]


def exact_int_gemm(rng, M, N, K, lim=4):
    """A[M,K], B[K,N] small integers: |A| <= lim, |B| <= lim, K*lim^2 <= 2048
    so every partial sum is an integer of magnitude <= 2048, exact in fp16."""
    A = rng.integers(-lim, lim + 1, size=(M, K)).astype(np.int64)
    B = rng.integers(-lim, lim + 1, size=(K, N)).astype(np.int64)
    C = A @ B
    assert np.abs(C).max() <= 2048 and K * lim * lim <= 2048
    return (A.astype(np.float16).view(np.uint16), B.astype(np.float16).view(np.uint16),
            C.astype(np.float16).view(np.uint16), C.astype(np.float32))


def main():
    with open(os.path.join(HERE, "blocks_known_answer.json"), "w") as f:
        json.dump({"source": "GGUF Q8_0/Q4_0 definitions; block sizes 34/18 bytes, 32 weights "
                             "(reference tests/test_gguf.cpp:16-34)",
                   "type_sizes": {"F32": 4, "F16": 2, "Q4_0": 18, "Q8_0": 34, "BF16": 2},
                   "block_sizes": {"F32": 1, "F16": 1, "Q4_0": 32, "Q8_0": 32},
                   "cases": known_answer_blocks()}, f, indent=1)
    rng = np.random.default_rng(20240601)
    arrays = {}
    for i, (M, N, K) in enumerate([(1, 8, 16), (3, 5, 7), (16, 33, 64), (1, 130, 128), (7, 64, 100)]):
        lim = 4 if K <= 128 else 2
        A, B, C16, C32 = exact_int_gemm(rng, M, N, K, lim)
        arrays[f"case{i}_shape"] = np.array([M, N, K], np.int32)
        arrays[f"case{i}_A"], arrays[f"case{i}_B"] = A, B
        arrays[f"case{i}_C16"], arrays[f"case{i}_C32"] = C16, C32
    np.savez(os.path.join(HERE, "gemm_exact_int.npz"), **arrays)
    print("wrote fixtures to", HERE)


if __name__ == "__main__":
    main()
