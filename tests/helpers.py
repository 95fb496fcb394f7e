"""Shared helpers for the tests: seeded inputs, descriptors, error metrics."""
from __future__ import annotations

import numpy as np


def contiguous_strides(shape):
    st, acc = [0] * len(shape), 1
    for i in range(len(shape) - 1, -1, -1):
        st[i] = acc
        acc *= int(shape[i])
    return st


def bcast_desc_uncollapsed(shape_a, shape_b):
    """(shape, sA, sB, sR) of a right-aligned broadcast, without collapsing (numpy rules)."""
    out = list(np.broadcast_shapes(tuple(shape_a), tuple(shape_b)))
    nd = len(out)

    def strides(sh):
        sh = [1] * (nd - len(sh)) + list(sh)
        cs = contiguous_strides(sh)
        return [0 if sh[i] == 1 and out[i] != 1 else cs[i] for i in range(nd)]

    return out, strides(shape_a), strides(shape_b), contiguous_strides(out)


def reduce_desc_uncollapsed(shape, axis, in_strides=None):
    """(shape_out, sOut, sIn), reduce_stride, n for reducing `axis` of a tensor."""
    in_strides = in_strides or contiguous_strides(shape)
    out_shape = [s for i, s in enumerate(shape) if i != axis]
    so = contiguous_strides(out_shape)
    si = [st for i, st in enumerate(in_strides) if i != axis]
    if not out_shape:
        out_shape, so, si = [1], [1], [1]
    return (out_shape, so, si), in_strides[axis], shape[axis]


def normwise_rel(x, ref):
    x = np.asarray(x, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(x - ref) / (den if den > 0 else 1.0))


def bits(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a)
    return a.view({1: np.uint8, 2: np.uint16, 4: np.uint32, 8: np.uint64}[a.dtype.itemsize])


def seeded_normal(rng, shape, dtype=np.float32):
    return rng.standard_normal(shape).astype(dtype)
