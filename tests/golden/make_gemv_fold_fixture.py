"""Writes gemv_fold_order.json: hand-built inputs on which only the summation
order of the reference gemv (src/kernels/gemm.cl:219-270) gives the recorded
output.

That kernel gives each group of 4 outputs 256 work items; item L accumulates
k = L, L+256, L+512, ... in ascending k with fma (gemm.cl:241-247), then the
group folds red[L] += red[L+s] for s = 128, 64, ..., 1 (gemm.cl:250-255) and
item 0 stores red[0] as half (gemm.cl:258-268).  In every case below each
nonzero product x[k]*W[k][0] is one of +2^24, -2^24 or +1 (fp16 operands
4096*4096, 4096*-4096, 1*1, all exact), and fp32 has no 2^24 + 1: RNE takes it
back to 2^24.  So whether the +1 survives depends only on which partial it is
added to first, i.e. on the order.  Each case records the reference order's
result (derived by hand in the comments) and what a plausible other order
gives, so a test can also check that the case tells the two apart.
Columns 1..3 of W are zero (outputs 0).

    python tests/golden/make_gemv_fold_fixture.py
"""
import json
import os

import numpy as np

H = lambda v: int(np.float16(v).view(np.uint16))   # fp16 bit pattern (exact for these values)
BIG = 4096.0                                        # 4096 * 4096 = 2^24

# (name, K, {k: (x_k, W[k][0])}, reference result, other order, its result)
CASES = [
    # lanes 0, 64, 128 hold +2^24, -2^24, +1.  s=128: red[0] = 2^24 + 1 -> 2^24;
    # red[64] = -2^24.  s=64: red[0] = 2^24 - 2^24 = 0; later strides add zeros.
    ("fold_pairs_stride_128_then_64", 256, {0: (BIG, BIG), 64: (BIG, -BIG), 128: (1.0, 1.0)},
     0.0, "partials summed in lane order 0..255", 1.0),
    # one lane, three terms k = 0, 256, 512: fma chain in ascending k:
    # 2^24, then 2^24 + 1 -> 2^24, then 2^24 - 2^24 = 0.
    ("ascending_k_inside_a_work_item", 768, {0: (BIG, BIG), 256: (1.0, 1.0), 512: (BIG, -BIG)},
     0.0, "k descending inside a work item (-2^24 + 1 = -16777215 exact, + 2^24 = 1)", 1.0),
    # strided partition: item 0 gets k = 0 and 256 (2^24 - 2^24 = 0), item 1
    # gets k = 1 (+1); the fold ends with red[0] = 0 + 1 = 1.
    ("strided_k_partition", 512, {0: (BIG, BIG), 1: (1.0, 1.0), 256: (BIG, -BIG)},
     1.0, "contiguous partition (item L takes k = 2L, 2L+1: item 0 = 2^24 + 1 -> 2^24, item 128 = -2^24)", 0.0),
    # items 0, 1, 2 hold 2^24, 1, -2^24.  s=2: red[0] = 2^24 - 2^24 = 0,
    # red[1] = 1; s=1: red[0] = 0 + 1 = 1.
    ("last_strides_2_then_1", 256, {0: (BIG, BIG), 1: (1.0, 1.0), 2: (BIG, -BIG)},
     1.0, "partials summed in lane order 0..255", 0.0),
]


def main():
    out = []
    for name, K, terms, want, other, other_val in CASES:
        N = 4
        x = np.zeros(K, np.float16)
        W = np.zeros((K, N), np.float16)
        for k, (xv, wv) in terms.items():
            x[k] = xv
            W[k, 0] = wv
        y = [H(want), 0, 0, 0]
        out.append({"name": name, "K": K, "N": N, "x": x.view(np.uint16).tolist(),
                    "W_kn": W.view(np.uint16).ravel().tolist(), "y_bits": y,
                    "other_order": other, "other_bits": [H(other_val), 0, 0, 0]})
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gemv_fold_order.json")
    with open(path, "w") as f:
        json.dump({"source": "src/kernels/gemm.cl:219-270 (gemv)", "cases": out}, f)
    print(f"wrote {path}: {len(out)} cases")


if __name__ == "__main__":
    main()
