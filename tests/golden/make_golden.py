"""Writes tests/golden/golden.npz: small seeded inputs with expected outputs computed by numpy.

Each expected output is fixed by mathematics independent of the oracle and of the kernels:
numpy float32 arithmetic is IEEE single (so broadcast ops are exact expectations), reductions
and contractions are evaluated in float64, argmax / argmin take numpy's first-index rule, and
casts use only in-range values.  Run from the repository root:

    python tests/golden/make_golden.py
"""
from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent / "golden.npz"


def main():
    rng = np.random.default_rng(20240601)
    g = {}
    # broadcast binary: [5, 7] op [1, 7], float32
    a = rng.standard_normal([5, 7]).astype(np.float32)
    b = rng.uniform(-2, 2, [1, 7]).astype(np.float32)
    b[0, 3] = a[2, 3]                      # an exact tie for max / min / equal
    g["bcast_a"], g["bcast_b"] = a, b
    g["bcast_add"], g["bcast_sub"] = a + b, a - b
    g["bcast_mul"], g["bcast_div"] = a * b, a / b
    g["bcast_max"] = np.where(a < b, b, a).astype(np.float32)
    g["bcast_min"] = np.where(b < a, b, a).astype(np.float32)
    g["bcast_eq"] = (a == b).astype(np.float32)
    # reductions over both axes of [6, 33] float32, with tied extrema
    x = rng.standard_normal([6, 33]).astype(np.float32)
    x[1, 20] = x[1].max()
    x[4, 2] = x[4].min()
    x[3, 5] = x[:, 5].max()
    g["red_x"] = x
    for ax in (0, 1):
        g[f"red_sum{ax}"] = x.astype(np.float64).sum(axis=ax)
        g[f"red_abs{ax}"] = np.abs(x.astype(np.float64)).sum(axis=ax)
        g[f"red_max{ax}"] = x.max(axis=ax)
        g[f"red_min{ax}"] = x.min(axis=ax)
        g[f"red_argmax{ax}"] = x.argmax(axis=ax).astype(np.int32)
        g[f"red_argmin{ax}"] = x.argmin(axis=ax).astype(np.int32)
    # batched matmul [2, 9, 13] x [13, 11] (B broadcast), float32 inputs, float64 result
    ma = rng.standard_normal([2, 9, 13]).astype(np.float32)
    mb = rng.standard_normal([13, 11]).astype(np.float32)
    g["mm_a"], g["mm_b"] = ma, mb
    g["mm_c"] = ma.astype(np.float64) @ mb.astype(np.float64)
    # conv: input [2, 6, 5, 3] NHWC, kernel [4, 3, 3, 3] OHWI, stride 1, pad 1, float64 result
    ci = rng.standard_normal([2, 6, 5, 3]).astype(np.float32)
    ck = rng.standard_normal([4, 3, 3, 3]).astype(np.float32)
    out = np.zeros([2, 6, 5, 4])
    pad = np.zeros([2, 8, 7, 3])
    pad[:, 1:7, 1:6, :] = ci
    for kh in range(3):
        for kw in range(3):
            out += np.einsum("nhwc,oc->nhwo", pad[:, kh:kh + 6, kw:kw + 5, :], ck[:, kh, kw, :].astype(np.float64))
    g["conv_in"], g["conv_k"], g["conv_out"] = ci, ck, out
    # casts of in-range values
    cv = (rng.uniform(-100, 100, 40)).astype(np.float32)
    g["cast_src"] = cv
    g["cast_i32"] = cv.astype(np.int32)                     # truncation toward zero
    g["cast_f16"] = cv.astype(np.float16).view(np.uint16)   # nearest even
    g["cast_u8"] = np.abs(cv).astype(np.uint8)
    g["cast_u8_src"] = np.abs(cv).astype(np.float32)
    np.savez(OUT, **g)
    print(f"wrote {OUT} ({len(g)} arrays)")


if __name__ == "__main__":
    main()
