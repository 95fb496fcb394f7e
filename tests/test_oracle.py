"""Pins the CPU oracle (oracle/oracle.c) against independent references.

The oracle restates the reference's CPU eval (see oracle/oracle.h for file:line).  Each test
checks it against something that does not share its code: numpy / torch arithmetic, closed
forms, hand-derived special cases of the reference's std::max / dtype_lowest semantics.
"""
import math

import numpy as np
import pytest
import torch

from helpers import bcast_desc_uncollapsed, bits, contiguous_strides, normwise_rel, reduce_desc_uncollapsed

FLT_MAX = np.float32(3.4028234663852886e38)


# ------------------------------------------------------------------ 16-bit conversions
def test_f16_to_f32_exhaustive(orc):
    h = np.arange(65536, dtype=np.uint16)
    got = orc.f16_bits_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(bits(got)[~nan], bits(ref)[~nan])


def test_f32_to_f16_matches_numpy_rne(orc):
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(2.0) ** rng.integers(-30, 20, 200000).astype(np.float32),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, np.inf, -np.inf, 2.0**-24, 2.0**-25,
                  3 * 2.0**-26, 2.0**-26, 1 + 2.0**-11, 1 + 3 * 2.0**-11, 2.0**-14, 2.0**-14 - 2.0**-25], np.float32),
    ])
    got = orc.f32_to_f16_bits(x)
    ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)
    nanbits = orc.f32_to_f16_bits(np.array([np.nan], np.float32))
    assert np.isnan(nanbits.view(np.float16)[0])


def test_f32_to_bf16_matches_torch_rne(orc):
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(100000) * 10.0 ** rng.integers(-30, 30, 100000)).astype(np.float32)
    x = np.concatenate([x, np.array([0.0, -0.0, np.inf, -np.inf, 1 + 2.0**-8, 1 + 3 * 2.0**-8], np.float32)])
    got = orc.f32_to_bf16_bits(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)


# ------------------------------------------------------------------ broadcast binary
SHAPES = [([4, 3, 5], [3, 1]), ([6, 1], [1, 7]), ([2, 3, 4, 5], [5]), ([1], [9]), ([5, 1, 3], [5, 4, 1])]


@pytest.mark.parametrize("sa,sb", SHAPES)
@pytest.mark.parametrize("op,fn", [(0, np.add), (1, np.subtract), (2, np.multiply), (3, np.divide)])
def test_bcast_f32_matches_numpy(orc, sa, sb, op, fn):
    rng = np.random.default_rng(2)
    a = rng.standard_normal(sa).astype(np.float32)
    b = (rng.standard_normal(sb) + 3).astype(np.float32)
    desc = bcast_desc_uncollapsed(sa, sb)
    total = int(np.prod(desc[0]))
    got = orc.bcast_binary(op, orc.F32, desc, total, a, b)
    ref = fn(a, b).astype(np.float32).ravel()
    assert np.array_equal(bits(got), bits(ref))


@pytest.mark.parametrize("op,fn", [(0, np.add), (1, np.subtract), (2, np.multiply), (3, np.divide)])
def test_bcast_f16_matches_numpy(orc, op, fn):
    rng = np.random.default_rng(3)
    a = (rng.standard_normal([8, 16]) * 100).astype(np.float16)
    b = (rng.standard_normal([16]) + 2).astype(np.float16)
    desc = bcast_desc_uncollapsed(a.shape, b.shape)
    got = orc.bcast_binary(op, orc.F16, desc, a.size, a.view(np.uint16), b.view(np.uint16))
    ref = fn(a, b).astype(np.float16).ravel()
    assert np.array_equal(got, ref.view(np.uint16))


@pytest.mark.parametrize("op", [0, 1, 2, 3])
def test_bcast_bf16_matches_torch(orc, op):
    rng = np.random.default_rng(4)
    a = torch.from_numpy(rng.standard_normal([8, 16]).astype(np.float32)).to(torch.bfloat16)
    b = torch.from_numpy((rng.standard_normal([16]) + 2).astype(np.float32)).to(torch.bfloat16)
    fn = [torch.add, torch.sub, torch.mul, torch.div][op]
    ref = fn(a, b).view(torch.int16).numpy().view(np.uint16).ravel()
    desc = bcast_desc_uncollapsed([8, 16], [16])
    got = orc.bcast_binary(op, orc.BF16, desc, 128, a.view(torch.int16).numpy().view(np.uint16),
                           b.view(torch.int16).numpy().view(np.uint16))
    assert np.array_equal(got, ref)


def test_bcast_max_min_select_semantics(orc):
    # std::max(a, b) = (a < b) ? b : a ; std::min(a, b) = (b < a) ? b : a  (Matrix.mm:13472, 14777)
    nan = np.float32(np.nan)
    a = np.array([1.0, 2.0, nan, 1.0, 0.0, -0.0, -np.inf, 3.0], np.float32)
    b = np.array([2.0, 1.0, 1.0, nan, -0.0, 0.0, -np.inf, 3.0], np.float32)
    desc = ([8], [1], [1], [1])
    mx_ = orc.bcast_binary(orc.MAX, orc.F32, desc, 8, a, b)
    mn_ = orc.bcast_binary(orc.MIN, orc.F32, desc, 8, a, b)
    # expected operand picked per lane: max -> b,a,a(NaN in a kept),a,a(+0),a(-0),a,a
    exp_max = np.array([b[0], a[1], a[2], a[3], a[4], a[5], a[6], a[7]], np.float32)
    exp_min = np.array([a[0], b[1], a[2], a[3], a[4], a[5], a[6], a[7]], np.float32)
    assert np.array_equal(bits(mx_), bits(exp_max))
    assert np.array_equal(bits(mn_), bits(exp_min))
    # on NaN-free, zero-free data it is numpy's maximum / minimum
    rng = np.random.default_rng(5)
    x = rng.standard_normal(1000).astype(np.float32)
    y = rng.standard_normal(1000).astype(np.float32)
    d = ([1000], [1], [1], [1])
    assert np.array_equal(orc.bcast_binary(orc.MAX, orc.F32, d, 1000, x, y), np.maximum(x, y))
    assert np.array_equal(orc.bcast_binary(orc.MIN, orc.F32, d, 1000, x, y), np.minimum(x, y))


INT_TYPES = [("I8", np.int8), ("I16", np.int16), ("I32", np.int32), ("I64", np.int64),
             ("U8", np.uint8), ("U16", np.uint16), ("U32", np.uint32), ("U64", np.uint64)]


@pytest.mark.parametrize("name,npt", INT_TYPES)
def test_bcast_int_wraps_like_numpy(orc, name, npt):
    code = getattr(orc, name)
    info = np.iinfo(npt)
    rng = np.random.default_rng(6)
    a = rng.integers(info.min, info.max, size=[7, 9], dtype=npt, endpoint=True)
    b = rng.integers(info.min, info.max, size=[9], dtype=npt, endpoint=True)
    desc = bcast_desc_uncollapsed(a.shape, b.shape)
    with np.errstate(over="ignore"):
        for op, fn in [(orc.ADD, np.add), (orc.SUB, np.subtract), (orc.MUL, np.multiply)]:
            got = orc.bcast_binary(op, code, desc, a.size, a, b)
            assert np.array_equal(got, fn(a, b).ravel()), (name, op)
    got = orc.bcast_binary(orc.MAX, code, desc, a.size, a, b)
    assert np.array_equal(got, np.maximum(a, b).ravel())
    got = orc.bcast_binary(orc.EQ, code, desc, a.size, a, b)
    assert np.array_equal(got, (a == b).astype(npt).ravel())


@pytest.mark.parametrize("name,npt", INT_TYPES)
def test_bcast_int_division_truncates(orc, name, npt):
    code = getattr(orc, name)
    info = np.iinfo(npt)
    vals = [info.min, info.min + 1, -7, -1, 0, 1, 7, 100, info.max] if info.min < 0 else [0, 1, 7, 100, info.max]
    vals = [v for v in vals if info.min <= v <= info.max]
    a = np.array([x for x in vals for _ in vals], dtype=npt)
    b = np.array([y for _ in vals for y in vals], dtype=npt)
    got = orc.bcast_binary(orc.DIV, code, ([a.size], [1], [1], [1]), a.size, a, b)
    exp = []
    for x, y in zip(a.tolist(), b.tolist()):
        if y == 0:
            q = 0                                   # arm64 sdiv/udiv: x / 0 == 0
        else:
            q = abs(x) // abs(y) * (1 if (x >= 0) == (y >= 0) else -1)
            if q > info.max:                        # MIN / -1 wraps to MIN
                q = info.min
        exp.append(q)
    assert np.array_equal(got, np.array(exp, dtype=npt))


def test_bcast_bool_truth_tables(orc):
    a = np.array([0, 0, 1, 1], np.uint8)
    b = np.array([0, 1, 0, 1], np.uint8)
    d = ([4], [1], [1], [1])
    table = {orc.ADD: [0, 1, 1, 1], orc.SUB: [0, 1, 1, 0], orc.MUL: [0, 0, 0, 1], orc.DIV: [0, 0, 0, 1],
             orc.MAX: [0, 1, 1, 1], orc.MIN: [0, 0, 0, 1], orc.EQ: [1, 0, 0, 1]}
    for op, exp in table.items():
        assert orc.bcast_binary(op, orc.BOOL, d, 4, a, b).tolist() == exp, op


def test_bcast_scalar_rank0(orc):
    a = np.array([3.5], np.float32)
    b = np.array([-1.25], np.float32)
    got = orc.bcast_binary(orc.MUL, orc.F32, ([], [], [], []), 1, a, b)
    assert got[0] == np.float32(3.5 * -1.25)


# ------------------------------------------------------------------ reductions
@pytest.mark.parametrize("shape,axis", [([37, 53], 1), ([37, 53], 0), ([4, 5, 6, 7], 2), ([4, 5, 6, 7], 0), ([300], 0)])
def test_reduce_f32_matches_numpy(orc, shape, axis):
    rng = np.random.default_rng(7)
    x = rng.standard_normal(shape).astype(np.float32)
    desc, rs, n = reduce_desc_uncollapsed(shape, axis)
    tot = int(np.prod(desc[0]))
    s = orc.reduce(orc.RSUM, orc.F32, rs, n, desc, tot, x)
    assert normwise_rel(s, x.astype(np.float64).sum(axis).ravel()) < 1e-6
    assert np.array_equal(orc.reduce(orc.RMAX, orc.F32, rs, n, desc, tot, x), x.max(axis).ravel())
    assert np.array_equal(orc.reduce(orc.RMIN, orc.F32, rs, n, desc, tot, x), x.min(axis).ravel())
    assert np.array_equal(orc.reduce(orc.RARGMAX, orc.F32, rs, n, desc, tot, x), x.argmax(axis).ravel())
    assert np.array_equal(orc.reduce(orc.RARGMIN, orc.F32, rs, n, desc, tot, x), x.argmin(axis).ravel())


def test_reduce_ties_first_index_like_numpy(orc):
    rng = np.random.default_rng(8)
    x = rng.integers(-3, 4, size=[64, 50]).astype(np.float32)   # many duplicate extrema
    desc, rs, n = reduce_desc_uncollapsed([64, 50], 1)
    assert np.array_equal(orc.reduce(orc.RARGMAX, orc.F32, rs, n, desc, 64, x), x.argmax(1))
    assert np.array_equal(orc.reduce(orc.RARGMIN, orc.F32, rs, n, desc, 64, x), x.argmin(1))


def test_reduce_special_values(orc):
    nan, inf = np.float32(np.nan), np.float32(np.inf)
    rows = np.array([
        [-inf, -inf, -inf, -inf],      # nothing beats -FLT_MAX: max -FLT_MAX, argmax 0
        [nan, 1.0, nan, 2.0],          # NaN never selected
        [0.0, -0.0, -1.0, -2.0],       # +0 first: stays +0
        [-0.0, 0.0, -1.0, -2.0],       # -0 first: stays -0
        [nan, nan, nan, nan],          # max -FLT_MAX, argmax 0
        [5.0, 7.0, 7.0, 1.0],          # first of the tie: 1
    ], np.float32)
    desc, rs, n = reduce_desc_uncollapsed([6, 4], 1)
    mx_ = orc.reduce(orc.RMAX, orc.F32, rs, n, desc, 6, rows)
    am = orc.reduce(orc.RARGMAX, orc.F32, rs, n, desc, 6, rows)
    assert bits(mx_).tolist() == bits(np.array([-FLT_MAX, 2.0, 0.0, -0.0, -FLT_MAX, 7.0], np.float32)).tolist()
    assert am.tolist() == [0, 3, 0, 0, 0, 1]
    mn = orc.reduce(orc.RMIN, orc.F32, rs, n, desc, 6, -rows)
    assert bits(mn).tolist() == bits(np.array([FLT_MAX, -2.0, -0.0, 0.0, FLT_MAX, -7.0], np.float32)).tolist()


def test_reduce_int_sum_wraps(orc):
    rng = np.random.default_rng(9)
    for name, npt in INT_TYPES:
        info = np.iinfo(npt)
        x = rng.integers(info.min, info.max, size=[5, 33], dtype=npt, endpoint=True)
        desc, rs, n = reduce_desc_uncollapsed([5, 33], 1)
        got = orc.reduce(orc.RSUM, getattr(orc, name), rs, n, desc, 5, x)
        assert np.array_equal(got, x.sum(1, dtype=npt)), name
        assert np.array_equal(orc.reduce(orc.RARGMAX, getattr(orc, name), rs, n, desc, 5, x), x.argmax(1))


def test_reduce_f16_literal_vs_f32_accumulator(orc):
    # 4096 ones: a half accumulator stalls at 2048 (2049 is not a half, ties to even);
    # the fp32 accumulator gives 4096.
    x = np.ones([1, 4096], np.float16).view(np.uint16)
    desc, rs, n = reduce_desc_uncollapsed([1, 4096], 1)
    lit = orc.reduce(orc.RSUM, orc.F16, rs, n, desc, 1, x, acc=orc.ACC_LITERAL)
    f32 = orc.reduce(orc.RSUM, orc.F16, rs, n, desc, 1, x, acc=orc.ACC_F32)
    assert lit.view(np.float16)[0] == 2048.0
    assert f32.view(np.float16)[0] == 4096.0


def test_reduce_empty_axis(orc):
    x = np.zeros([3, 0], np.float32)
    desc = ([3], [1], [0])
    assert orc.reduce(orc.RSUM, orc.F32, 1, 0, desc, 3, np.zeros(1, np.float32)).tolist() == [0, 0, 0]
    assert bits(orc.reduce(orc.RMAX, orc.F32, 1, 0, desc, 3, np.zeros(1, np.float32))).tolist() == \
        bits(np.full(3, -FLT_MAX, np.float32)).tolist()
    del x


# ------------------------------------------------------------------ matmul
def _mm_desc(batch, M, N, K, b_broadcast):
    shape = [batch, M, N]
    sA = [M * K, K, 1]
    sBt = [0 if b_broadcast else N * K, K, 1]
    sC = [M * N, N, 1]
    return shape, sA, sBt, sC


@pytest.mark.parametrize("bcast", [True, False])
def test_matmul_f32_matches_numpy(orc, bcast):
    rng = np.random.default_rng(10)
    batch, M, N, K = 3, 17, 13, 33
    A = rng.standard_normal([batch, M, K]).astype(np.float32)
    Bt = rng.standard_normal([1 if bcast else batch, N, K]).astype(np.float32)
    C = orc.batched_matmul(orc.F32, _mm_desc(batch, M, N, K, bcast), K, A, Bt, batch * M * N)
    ref = np.matmul(A.astype(np.float64), np.swapaxes(Bt.astype(np.float64), -1, -2))
    assert normwise_rel(C, ref) < 1e-6


def test_matmul_f16_accumulators(orc):
    rng = np.random.default_rng(11)
    M, N, K = 16, 16, 2048
    A = (rng.standard_normal([1, M, K]) / math.sqrt(K)).astype(np.float16)
    Bt = rng.standard_normal([1, N, K]).astype(np.float16)
    ref = A.astype(np.float64)[0] @ Bt.astype(np.float64)[0].T
    desc = _mm_desc(1, M, N, K, False)
    f32 = orc.batched_matmul(orc.F16, desc, K, A.view(np.uint16), Bt.view(np.uint16), M * N, acc=orc.ACC_F32)
    lit = orc.batched_matmul(orc.F16, desc, K, A.view(np.uint16), Bt.view(np.uint16), M * N, acc=orc.ACC_LITERAL)
    e32 = normwise_rel(f32.view(np.float16), ref)
    elit = normwise_rel(lit.view(np.float16), ref)
    assert e32 < 1e-3           # one rounding to half
    assert elit > e32           # per-step half rounding is visibly worse


def test_matmul_int_exact(orc):
    rng = np.random.default_rng(12)
    A = rng.integers(-50, 50, size=[2, 5, 7]).astype(np.int32)
    Bt = rng.integers(-50, 50, size=[2, 3, 7]).astype(np.int32)
    C = orc.batched_matmul(orc.I32, _mm_desc(2, 5, 3, 7, False), 7, A, Bt, 30)
    assert np.array_equal(C.reshape(2, 5, 3), np.matmul(A, np.swapaxes(Bt, 1, 2)))


# ------------------------------------------------------------------ convolution
def _conv_ref_torch(x_nhwc, w_ohwi, stride, pad, dil, groups, flip, dil_lhs, out_spatial):
    """torch conv in float64 on NCHW, with input dilation done by zero insertion."""
    ns = x_nhwc.ndim - 2
    x = torch.from_numpy(x_nhwc.astype(np.float64)).movedim(-1, 1)
    w = torch.from_numpy(w_ohwi.astype(np.float64)).movedim(-1, 1)
    if flip:
        w = torch.flip(w, dims=list(range(2, 2 + ns)))
    if any(d > 1 for d in dil_lhs):
        shp = list(x.shape[:2]) + [(s - 1) * d + 1 for s, d in zip(x.shape[2:], dil_lhs)]
        xd = torch.zeros(shp, dtype=x.dtype)
        sl = (slice(None), slice(None)) + tuple(slice(None, None, d) for d in dil_lhs)
        xd[sl] = x
        x = xd
    # the reference pads pad_lo on the low side and as much as the output needs on the high side
    hi = [max(0, (o - 1) * s + (k - 1) * d + 1 - (xs + p)) for o, s, k, d, xs, p in
          zip(out_spatial, stride, w.shape[2:], dil, x.shape[2:], pad)]
    padspec = []
    for p, h in reversed(list(zip(pad, hi))):
        padspec += [p, h]
    x = torch.nn.functional.pad(x, padspec)
    fn = {1: torch.nn.functional.conv1d, 2: torch.nn.functional.conv2d, 3: torch.nn.functional.conv3d}[ns]
    y = fn(x, w, stride=stride, dilation=dil, groups=groups)
    sl = (slice(None), slice(None)) + tuple(slice(0, o) for o in out_spatial)
    return y[sl].movedim(1, -1).contiguous().numpy()


CONV_CASES = [
    # (N, spatial, C, O, ksize, stride, pad, dil, groups, flip, dil_lhs)
    (2, [9, 8], 6, 4, [3, 3], [1, 1], [1, 1], [1, 1], 1, False, [1, 1]),
    (2, [10, 10], 8, 6, [1, 1], [2, 2], [0, 0], [1, 1], 1, False, [1, 1]),
    (1, [11, 9], 4, 4, [3, 2], [2, 1], [2, 0], [2, 1], 2, False, [1, 1]),
    (1, [7, 7], 3, 2, [3, 3], [1, 1], [1, 1], [1, 1], 1, True, [1, 1]),
    (1, [5, 6], 2, 3, [3, 3], [1, 1], [2, 2], [1, 1], 1, False, [2, 2]),
    (2, [13], 4, 5, [3], [2], [1], [1], 1, False, [1]),
    (1, [5, 4, 6], 3, 2, [3, 1, 3], [1, 1, 2], [1, 0, 1], [1, 1, 1], 1, False, [1, 1, 1]),
]


def _conv_out_shape(spatial, ksize, stride, pad, dil, dil_lhs):
    out = []
    for s, k, st, p, d, dl in zip(spatial, ksize, stride, pad, dil, dil_lhs):
        span = dl * (s - 1) + 1 + 2 * p - (d * (k - 1) + 1)
        out.append(span // st + 1)
    return out


@pytest.mark.parametrize("case", CONV_CASES)
def test_conv_matches_torch(orc, case):
    N, sp, C, O, ks, st, pad, dil, groups, flip, dl = case
    rng = np.random.default_rng(13)
    x = rng.standard_normal([N, *sp, C]).astype(np.float32)
    w = rng.standard_normal([O, *ks, C // groups]).astype(np.float32)
    osp = _conv_out_shape(sp, ks, st, pad, dil, dl)
    out_shape = [N, *osp, O]
    got = orc.conv(orc.F32, list(x.shape), list(w.shape), out_shape, contiguous_strides(x.shape),
                   contiguous_strides(w.shape), contiguous_strides(out_shape), pad, st, dil, dl, groups, flip,
                   x, w, int(np.prod(out_shape)))
    ref = _conv_ref_torch(x, w, st, pad, dil, groups, flip, dl, osp)
    assert normwise_rel(got, ref) < 1e-6


def test_conv_strided_views_equal_contiguous(orc):
    # NCHW-stored tensors fed as NHWC views (the reference's transpose(0,2,3,1))
    rng = np.random.default_rng(14)
    x_nchw = rng.standard_normal([2, 5, 7, 6]).astype(np.float32)
    w_oihw = rng.standard_normal([3, 5, 3, 3]).astype(np.float32)
    in_shape, k_shape, out_shape = [2, 7, 6, 5], [3, 3, 3, 5], [2, 7, 6, 3]
    xs = contiguous_strides(x_nchw.shape)
    ws = contiguous_strides(w_oihw.shape)
    in_strides = [xs[0], xs[2], xs[3], xs[1]]
    k_strides = [ws[0], ws[2], ws[3], ws[1]]
    common = (out_shape, None, [1, 1], [1, 1], [1, 1], [1, 1], 1, False)
    got = orc.conv(orc.F32, in_shape, k_shape, out_shape, in_strides, k_strides, contiguous_strides(out_shape),
                   [1, 1], [1, 1], [1, 1], [1, 1], 1, False, x_nchw, w_oihw, 2 * 7 * 6 * 3)
    x_nhwc = np.ascontiguousarray(x_nchw.transpose(0, 2, 3, 1))
    w_ohwi = np.ascontiguousarray(w_oihw.transpose(0, 2, 3, 1))
    ref = orc.conv(orc.F32, in_shape, k_shape, out_shape, contiguous_strides(in_shape), contiguous_strides(k_shape),
                   contiguous_strides(out_shape), [1, 1], [1, 1], [1, 1], [1, 1], 1, False, x_nhwc, w_ohwi,
                   2 * 7 * 6 * 3)
    assert np.array_equal(got, ref)
    del common


def test_conv_1x1_is_matmul(orc):
    rng = np.random.default_rng(15)
    x = rng.integers(-5, 5, size=[2, 4, 4, 6]).astype(np.int32)
    w = rng.integers(-5, 5, size=[5, 1, 1, 6]).astype(np.int32)
    out_shape = [2, 4, 4, 5]
    got = orc.conv(orc.I32, list(x.shape), list(w.shape), out_shape, contiguous_strides(x.shape),
                   contiguous_strides(w.shape), contiguous_strides(out_shape), [0, 0], [1, 1], [1, 1], [1, 1], 1,
                   False, x, w, 160)
    assert np.array_equal(got.reshape(32, 5), x.reshape(32, 6) @ w.reshape(5, 6).T)


# ------------------------------------------------------------------ strided copy
def test_copy_transpose_and_cast(orc):
    rng = np.random.default_rng(16)
    src = rng.standard_normal([4, 5, 6]).astype(np.float32) * 10
    # dst = src.transpose(2, 0, 1) as float16, contiguous
    shape = [6, 4, 5]
    s_src = [1, 30, 6]
    dst = np.zeros(120, np.uint16)
    orc.copy_strided(orc.F16, orc.F32, shape, contiguous_strides(shape), s_src, dst, src)
    assert np.array_equal(dst, src.transpose(2, 0, 1).astype(np.float16).ravel().view(np.uint16))
    dsti = np.zeros(120, np.int32)
    orc.copy_strided(orc.I32, orc.F32, shape, contiguous_strides(shape), s_src, dsti, src)
    assert np.array_equal(dsti, np.trunc(src.transpose(2, 0, 1)).astype(np.int32).ravel())


# ------------------------------------------------------------------ complex64
U32 = 2.0 ** -24      # unit roundoff of float32


def _c64(rng, n, scale=4.0):
    z = (rng.standard_normal(n) * scale + 1j * rng.standard_normal(n) * scale).astype(np.complex64)
    return z


def _bin(orc, op, a, b):
    n = a.size
    return orc.bcast_binary(op, orc.C64, ([n], [1], [1], [1]), n, a, b)


def test_complex_add_sub_are_componentwise_float32(orc):
    """Add / Sub are per-part float32 sums (complex.h:28-34): numpy's complex64 arithmetic."""
    rng = np.random.default_rng(40)
    a, b = _c64(rng, 4096), _c64(rng, 4096)
    assert np.array_equal(bits(_bin(orc, orc.ADD, a, b)), bits(a + b))
    assert np.array_equal(bits(_bin(orc, orc.SUB, a, b)), bits(a - b))


def test_complex_mul_div_within_rounding_of_exact(orc):
    """Mul / Div against complex128 arithmetic on the same float32 inputs: each part within the
    rounding the formula allows (2u of |a||c| + |b||d| for the product, 6u of
    (|a| + |b|)(|c| + |d|) / |rhs|^2 for the quotient).  A swapped part, a wrong sign or a dropped
    term is off by O(1)."""
    rng = np.random.default_rng(41)
    a, b = _c64(rng, 8192), _c64(rng, 8192)
    A, B = a.astype(np.complex128), b.astype(np.complex128)
    got = _bin(orc, orc.MUL, a, b).astype(np.complex128)
    ex = A * B
    sr = np.abs(A.real * B.real) + np.abs(A.imag * B.imag)
    si = np.abs(A.imag * B.real) + np.abs(A.real * B.imag)
    assert np.all(np.abs(got.real - ex.real) <= 2 * U32 * sr)
    assert np.all(np.abs(got.imag - ex.imag) <= 2 * U32 * si)
    got = _bin(orc, orc.DIV, a, b).astype(np.complex128)
    ex = A / B
    bound = 6 * U32 * (np.abs(A.real) + np.abs(A.imag)) * (np.abs(B.real) + np.abs(B.imag)) / np.abs(B) ** 2
    assert np.all(np.abs(got.real - ex.real) <= bound)
    assert np.all(np.abs(got.imag - ex.imag) <= bound)


def test_complex_exact_special_cases(orc):
    """z * 1 = z, z * i = (-b, a), z / 1 = z, i * i = -1: exact in the formula."""
    rng = np.random.default_rng(42)
    z = _c64(rng, 1000)
    z = z[(z.real != 0) & (z.imag != 0)]
    one = np.ones(z.size, np.complex64)
    i = np.full(z.size, 1j, np.complex64)
    assert np.array_equal(bits(_bin(orc, orc.MUL, z, one)), bits(z))
    assert np.array_equal(bits(_bin(orc, orc.DIV, z, one)), bits(z))
    want = (-z.imag + 1j * z.real).astype(np.complex64)
    assert np.array_equal(bits(_bin(orc, orc.MUL, z, i)), bits(want))
    assert _bin(orc, orc.MUL, i[:1], i[:1])[0] == -1


def test_complex_mul_fuses_the_first_product(orc):
    """(a + bi)(c + di) = (a, b) c + (-b, a) d with the first product fused: im of z * conj(z) is
    fma(b, a, -fl(a b)) = a b - fl(a b), the exact rounding error of a b (the other fusion
    gives its negative, an unfused product gives 0)."""
    rng = np.random.default_rng(43)
    z = _c64(rng, 2000)
    got = _bin(orc, orc.MUL, z, np.conj(z))
    ab = z.real.astype(np.float64) * z.imag.astype(np.float64)     # exact: 24 + 24 bits
    err = ab - (z.real * z.imag).astype(np.float64)
    assert np.array_equal(got.imag.astype(np.float64), err.astype(np.float32).astype(np.float64))
    assert np.any(err != 0)


def test_complex_div_is_unscaled(orc):
    """Division by c c + d d without scaling (complex.h:50-52): |rhs| past ~1.8e19 overflows the
    denominator to inf and gives 0; |rhs| below ~1e-23 underflows it to 0 and gives inf.  A scaled
    (Smith) division would return 1e-20 and 1e30."""
    a = np.array([1 + 1j, 1 + 0j], np.complex64)
    b = np.array([1e20 + 0j, 1e-30 + 0j], np.complex64)
    got = _bin(orc, orc.DIV, a, b)
    assert got[0] == 0
    assert np.isinf(got[1].real)


def test_complex_rejects_ordering_ops(orc):
    a = np.ones(4, np.complex64)
    for op in (orc.MAX, orc.MIN, orc.EQ):
        with pytest.raises(ValueError):
            _bin(orc, op, a, a)


def test_copy_complex_moves_bits_and_casts_from_real(orc):
    """complex64 -> complex64 moves the 8 bytes (a transposed view here); a real dtype -> complex64
    is (float(v), 0), numpy's astype for the dtypes it converts exactly; complex64 -> real has no
    cast."""
    rng = np.random.default_rng(44)
    z = _c64(rng, 120).reshape(4, 5, 6)
    z[0, 0, 0] = complex(np.nan, -0.0)
    dst = np.zeros(120, np.complex64)
    orc.copy_strided(orc.C64, orc.C64, [6, 4, 5], contiguous_strides([6, 4, 5]), [1, 30, 6], dst, z)
    assert np.array_equal(bits(dst), bits(z.transpose(2, 0, 1).ravel()))
    for code, x in ((orc.F32, rng.standard_normal(64).astype(np.float32)),
                    (orc.F16, rng.standard_normal(64).astype(np.float16)),
                    (orc.I32, rng.integers(-2**31, 2**31 - 1, 64, dtype=np.int32)),
                    (orc.U8, rng.integers(0, 255, 64, dtype=np.uint8)),
                    (orc.BOOL, rng.integers(0, 2, 64).astype(np.bool_))):
        out = np.zeros(64, np.complex64)
        orc.copy_strided(orc.C64, code, [64], [1], [1], out, x)
        assert np.array_equal(bits(out), bits(x.astype(np.complex64))), code
    x = rng.integers(-2**63, 2**63 - 1, 64, dtype=np.int64)
    out = np.zeros(64, np.complex64)
    f = np.zeros(64, np.float32)
    orc.copy_strided(orc.C64, orc.I64, [64], [1], [1], out, x)
    orc.copy_strided(orc.F32, orc.I64, [64], [1], [1], f, x)
    assert np.array_equal(bits(out.real.copy()), bits(f)) and not out.imag.any()
    with pytest.raises(ValueError):
        orc.copy_strided(orc.F32, orc.C64, [4], [1], [1], np.zeros(4, np.float32), np.zeros(4, np.complex64))
