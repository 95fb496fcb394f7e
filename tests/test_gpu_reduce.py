"""GPU parity: Sum / Max / Min / ArgMax / ArgMin vs the oracle.

Max / Min / ArgMax / ArgMin and integer sums are bit-exact; fp32 sums satisfy
|gpu - cpu| <= 1e-4 * sum|x| per output (and normwise <= 1e-4); 16-bit float sums are
checked against the oracle's fp32-accumulator mode (one rounding at the end).
"""
import numpy as np
import pytest

from helpers import bits, contiguous_strides, normwise_rel

pytestmark = pytest.mark.gpu

SUM_TOL = 1e-4


def reduce_desc(mx, shape, axis, in_strides=None, keepdims=False):
    in_strides = in_strides or contiguous_strides(shape)
    if keepdims:
        out_shape = [1 if i == axis else s for i, s in enumerate(shape)]
    else:
        out_shape = [s for i, s in enumerate(shape) if i != axis]
    desc = mx.collapse_dims_reduce2(shape, contiguous_strides(out_shape), in_strides, axis,
                                    keep_dims=False, outer_collapsed=not keepdims)
    total = int(np.prod(out_shape)) if out_shape else 1
    return desc, in_strides[axis], shape[axis], total


def run_reduce(mx, orc, op, code, x_flat, shape, axis, in_strides=None, keepdims=False, acc=None):
    desc, rs, n, total = reduce_desc(mx, shape, axis, in_strides, keepdims)
    X = mx.DeviceBuffer(max(x_flat.nbytes, 16))
    X.upload(x_flat.view(np.uint8))
    out_dt = np.int32 if op in (mx.RED_ARGMAX, mx.RED_ARGMIN) else x_flat.dtype
    O = mx.DeviceBuffer(max(total, 1) * np.dtype(out_dt).itemsize)
    wsb = mx.reduce_workspace_bytes(op, code, rs, n, desc)
    W = mx.DeviceBuffer(wsb) if wsb else None
    if W:
        W.fill_bytes(0)
    mx.launch_reduce(op, code, rs, n, desc, O.ptr, X.ptr, W.ptr if W else 0, wsb)
    mx.sync()
    got = O.download(out_dt, total)
    if W:
        # split plans: a second launch on the same workspace gives the same bits
        O2 = mx.DeviceBuffer(max(total, 1) * np.dtype(out_dt).itemsize)
        mx.launch_reduce(op, code, rs, n, desc, O2.ptr, X.ptr, W.ptr, wsb)
        mx.sync()
        assert np.array_equal(bits(O2.download(out_dt, total)), bits(got))
    ref = orc.reduce(op, code, rs, n, desc, total, x_flat, acc=orc.ACC_F32 if acc is None else acc)
    return got, ref, desc, rs, n


def check_sum(got, ref, x_abs_sum):
    g = got.astype(np.float64)
    r = ref.astype(np.float64)
    assert np.all(np.abs(g - r) <= SUM_TOL * np.maximum(x_abs_sum, 1e-30) + 1e-30)
    assert normwise_rel(g, r) <= SUM_TOL


def abs_sum(mx, x_flat, shape, axis, in_strides=None):
    in_strides = in_strides or contiguous_strides(shape)
    view = np.lib.stride_tricks.as_strided(x_flat.astype(np.float64),
                                           shape=shape, strides=[s * 8 for s in in_strides])
    return np.abs(view).sum(axis).ravel()


def inject_ties(rng, x, axis, frac=0.3, minimum=False):
    """Copy each chosen row's extremum to 1-3 more random positions (30% of rows)."""
    xm = np.moveaxis(x, axis, -1)
    rows = xm.reshape(-1, xm.shape[-1])
    for r in np.nonzero(rng.random(rows.shape[0]) < frac)[0]:
        v = rows[r].min() if minimum else rows[r].max()
        rows[r, rng.integers(0, rows.shape[1], rng.integers(1, 4))] = v
    return np.ascontiguousarray(np.moveaxis(rows.reshape(xm.shape), -1, axis))


OPS = ["RED_SUM", "RED_MAX", "RED_MIN", "RED_ARGMAX", "RED_ARGMIN"]


@pytest.mark.parametrize("axis", [1, 0])
@pytest.mark.parametrize("opn", OPS)
def test_reductions_256x65536(mx, orc, axis, opn):
    """X[256,65536] ~ N(0,1), seed 0, 30% of rows with duplicated extrema (the reductions workload)."""
    op = getattr(mx, opn)
    rng = np.random.default_rng(0)
    x = rng.standard_normal([256, 65536]).astype(np.float32)
    x = inject_ties(rng, x, axis, minimum=op in (mx.RED_MIN, mx.RED_ARGMIN))
    got, ref, *_ = run_reduce(mx, orc, op, mx.FLOAT32, x.ravel(), [256, 65536], axis)
    if op == mx.RED_SUM:
        check_sum(got, ref, np.abs(x.astype(np.float64)).sum(axis))
    else:
        assert np.array_equal(bits(got), bits(ref))


@pytest.mark.parametrize("opn", OPS)
def test_reshaped_chain_axes_3_then_1(mx, orc, opn):
    """X.reshape(64,4,4096,16) reduced over axis 3, then axis 1 (the non-contiguous split)."""
    op = getattr(mx, opn)
    rng = np.random.default_rng(1)
    x = rng.standard_normal([64, 4, 4096, 16]).astype(np.float32)
    got3, ref3, desc, *_ = run_reduce(mx, orc, op, mx.FLOAT32, x.ravel(), [64, 4, 4096, 16], 3)
    assert desc == [[1048576], [1], [16]]
    if op == mx.RED_SUM:
        check_sum(got3, ref3, np.abs(x.astype(np.float64)).sum(3).ravel())
    else:
        assert np.array_equal(bits(got3), bits(ref3))
    if op in (mx.RED_ARGMAX, mx.RED_ARGMIN):
        # arg-reductions take one axis: run axis 1 of the original tensor's [64,4,4096] slice
        y = np.ascontiguousarray(x[..., 0])
    else:
        y = got3.reshape(64, 4, 4096)
    got1, ref1, desc1, *_ = run_reduce(mx, orc, op, mx.FLOAT32, y.ravel(), [64, 4, 4096], 1)
    assert desc1 == [[64, 4096], [4096, 1], [16384, 1]]
    if op == mx.RED_SUM:
        check_sum(got1, ref1, np.abs(y.astype(np.float64)).sum(1).ravel())
    else:
        assert np.array_equal(bits(got1), bits(ref1))


@pytest.mark.parametrize("opn", ["RED_ARGMAX", "RED_ARGMIN", "RED_MAX", "RED_MIN", "RED_SUM"])
def test_reshaped_axis1_full(mx, orc, opn):
    """Every reduction over axis 1 of the whole X.reshape(64,4,4096,16) (the arg-reductions' second
    axis of the workload), with 30% of the axis-1 rows carrying duplicated extrema (first index
    wins), against the oracle."""
    op = getattr(mx, opn)
    rng = np.random.default_rng(2)
    x = rng.standard_normal([64, 4, 4096, 16]).astype(np.float32)
    x = inject_ties(rng, x, 1, minimum=op in (mx.RED_MIN, mx.RED_ARGMIN))
    got, ref, desc, *_ = run_reduce(mx, orc, op, mx.FLOAT32, x.ravel(), [64, 4, 4096, 16], 1)
    assert desc == [[64, 65536], [65536, 1], [262144, 1]]
    if op == mx.RED_SUM:
        check_sum(got, ref, np.abs(x.astype(np.float64)).sum(1).ravel())
    else:
        assert np.array_equal(bits(got), bits(ref))
        if op in (mx.RED_ARGMAX, mx.RED_ARGMIN):      # first index of the extremum, as numpy's
            npf = np.argmax if op == mx.RED_ARGMAX else np.argmin
            assert np.array_equal(got, npf(x, axis=1).ravel().astype(np.int32))


def test_add_rowsum_sum(mx, orc):
    rng = np.random.default_rng(0)
    a = rng.standard_normal([4096, 1024]).astype(np.float32)
    b = rng.uniform(-1, 1, [1, 1024]).astype(np.float32)
    c = (a + b).astype(np.float32)
    got, ref, *_ = run_reduce(mx, orc, mx.RED_SUM, mx.FLOAT32, c.ravel(), [4096, 1024], 1)
    check_sum(got, ref, np.abs(c.astype(np.float64)).sum(1))


@pytest.mark.parametrize("shape,axis", [([3, 5], 1), ([7, 2], 1), ([9, 40], 1), ([11, 200], 1), ([5, 3000], 1),
                                        ([2, 50000], 1), ([37, 53], 0), ([4, 5, 6, 7], 2), ([4, 5, 6, 7], 0),
                                        ([1, 1], 0), ([6, 1, 8], 1), ([3, 4, 5], 2), ([3000, 8], 0),
                                        ([20000, 12], 0), ([700, 36], 0), ([5, 100003], 1), ([129, 1000], 0)])
@pytest.mark.parametrize("opn", OPS)
def test_plans_f32(mx, orc, shape, axis, opn):
    """Covers every plan: L-lane rows, block + finalize, columns with and without chunks."""
    op = getattr(mx, opn)
    rng = np.random.default_rng(2)
    x = np.round(rng.standard_normal(shape) * 3).astype(np.float32)   # many ties and +-0
    x[rng.random(shape) < 0.1] *= -0.0
    got, ref, *_ = run_reduce(mx, orc, op, mx.FLOAT32, x.ravel(), shape, axis)
    if op == mx.RED_SUM:
        check_sum(got, ref, abs_sum(mx, x.ravel(), shape, axis))
    else:
        assert np.array_equal(bits(got), bits(ref))


@pytest.mark.parametrize("keepdims", [False, True])
def test_keepdims_and_strided_input(mx, orc, keepdims):
    rng = np.random.default_rng(3)
    base = rng.standard_normal([24, 36]).astype(np.float32)
    # transposed view [36, 24] with strides [1, 36]
    for op in (mx.RED_MAX, mx.RED_ARGMIN, mx.RED_SUM):
        for axis in (0, 1):
            got, ref, *_ = run_reduce(mx, orc, op, mx.FLOAT32, base.ravel(), [36, 24], axis, in_strides=[1, 36],
                                      keepdims=keepdims)
            if op == mx.RED_SUM:
                check_sum(got, ref, np.abs(base.T.astype(np.float64)).sum(axis).ravel())
            else:
                assert np.array_equal(bits(got), bits(ref))


def test_special_rows(mx, orc):
    nan, inf = np.nan, np.inf
    rows = np.full([8, 1000], -inf, np.float32)
    rows[1, 500] = nan
    rows[2, :] = nan
    rows[2, 999] = -3.0
    rows[3, :] = 0.0
    rows[3, 7] = -0.0
    rows[4, :] = -0.0
    rows[4, 900] = 0.0
    rows[5, ::3] = 5.0
    rows[6, :] = -3.4028234663852886e38
    rows[7, :] = np.linspace(-1, 1, 1000, dtype=np.float32)
    for op in (mx.RED_MAX, mx.RED_MIN, mx.RED_ARGMAX, mx.RED_ARGMIN):
        for x in (rows, -rows):
            got, ref, *_ = run_reduce(mx, orc, op, mx.FLOAT32, np.ascontiguousarray(x).ravel(), [8, 1000], 1)
            assert np.array_equal(bits(got), bits(ref)), op
            gotc, refc, *_ = run_reduce(mx, orc, op, mx.FLOAT32, np.ascontiguousarray(x.T).ravel(), [1000, 8], 0)
            assert np.array_equal(bits(gotc), bits(refc)), op


INT_DTYPES = ["INT32", "INT8", "INT16", "INT64", "UINT8", "UINT16", "UINT32", "UINT64", "BOOL"]


@pytest.mark.parametrize("dt", INT_DTYPES)
@pytest.mark.parametrize("opn", OPS)
def test_integer_dtypes_exact(mx, orc, dt, opn):
    code, op = getattr(mx, dt), getattr(mx, opn)
    npt = mx.NP_DTYPE[code]
    rng = np.random.default_rng(4)
    for shape, axis in [([16, 700], 1), ([300, 40], 0), ([5, 9000], 1)]:
        if code == mx.BOOL:
            x = rng.integers(0, 2, size=shape).astype(np.bool_)
        else:
            info = np.iinfo(npt)
            x = rng.integers(info.min, info.max, size=shape, dtype=npt, endpoint=True)
        got, ref, *_ = run_reduce(mx, orc, op, code, x.ravel(), shape, axis)
        assert np.array_equal(bits(got), bits(ref)), (dt, opn, shape, axis)


@pytest.mark.parametrize("dt", ["FLOAT16", "BFLOAT16"])
@pytest.mark.parametrize("opn", OPS)
def test_half_dtypes(mx, orc, dt, opn):
    code, op = getattr(mx, dt), getattr(mx, opn)
    rng = np.random.default_rng(5)
    for shape, axis in [([16, 4000], 1), ([300, 48], 0), ([8, 64], 1)]:
        xf = np.round(rng.standard_normal(shape) * 8).astype(np.float32)
        if code == mx.FLOAT16:
            x = xf.astype(np.float16)
        else:
            from oracle.oracle import f32_to_bf16_bits
            x = f32_to_bf16_bits(xf)
        got, ref, *_ = run_reduce(mx, orc, op, code, x.ravel(), shape, axis)
        if op == mx.RED_SUM:
            g = got.astype(np.float32) if code == mx.FLOAT16 else (got.astype(np.uint32) << 16).view(np.float32)
            r = ref.astype(np.float32) if code == mx.FLOAT16 else (ref.astype(np.uint32) << 16).view(np.float32)
            # integer-valued inputs: fp32 partial sums are exact, so both round the same exact sum
            assert np.array_equal(g, r)
        else:
            assert np.array_equal(bits(got), bits(ref))


def test_empty_reduced_axis(mx, orc):
    # shape[axis] == 0: sum 0, max -FLT_MAX, argmax 0, as the reference's empty loops give
    desc = [[3], [1], [0]]
    X = mx.DeviceBuffer(16)
    for op, exp in [(mx.RED_SUM, [0.0] * 3), (mx.RED_MAX, [-3.4028234663852886e38] * 3), (mx.RED_ARGMAX, [0] * 3)]:
        dt = np.int32 if op == mx.RED_ARGMAX else np.float32
        O = mx.DeviceBuffer(12)
        mx.launch_reduce(op, mx.FLOAT32, 1, 0, desc, O.ptr, X.ptr)
        mx.sync()
        assert O.download(dt, 3).tolist() == np.array(exp, dt).tolist()


def test_workspace_too_small_is_an_error(mx):
    # 4 rows of 2^20: too few outputs to cover the CUs, so each row is split over blocks
    desc = [[4], [1], [1 << 20]]
    nb = mx.reduce_workspace_bytes(mx.RED_SUM, mx.FLOAT32, 1, 1 << 20, desc)
    assert nb > 0
    X = mx.DeviceBuffer(4 * (1 << 20) * 4)
    O = mx.DeviceBuffer(4 * 4)
    with pytest.raises(mx.MatrixAMDError, match="workspace"):
        mx.launch_reduce(mx.RED_SUM, mx.FLOAT32, 1, 1 << 20, desc, O.ptr, X.ptr, 0, 0)


@pytest.mark.parametrize("opn", OPS)
def test_split_rows_few_outputs(mx, orc, opn):
    """Few long rows: the axis is split over blocks and the last block combines."""
    op = getattr(mx, opn)
    rng = np.random.default_rng(6)
    x = np.round(rng.standard_normal([3, 1 << 20]) * 4).astype(np.float32)
    got, ref, *_ = run_reduce(mx, orc, op, mx.FLOAT32, x.ravel(), [3, 1 << 20], 1)
    if op == mx.RED_SUM:
        check_sum(got, ref, np.abs(x.astype(np.float64)).sum(1))
    else:
        assert np.array_equal(bits(got), bits(ref))


@pytest.mark.parametrize("dt,shape,axis", [
    ("FLOAT32", [5000, 16], 1), ("FLOAT32", [333, 8], 1), ("FLOAT32", [777, 12], 1), ("FLOAT32", [100, 4], 1),
    ("FLOAT16", [900, 32], 1), ("BFLOAT16", [257, 24], 1), ("INT8", [300, 64], 1), ("INT64", [500, 6], 1),
    ("FLOAT32", [2, 300000], 0), ("FLOAT32", [7, 40000], 0), ("FLOAT32", [8, 36], 0), ("FLOAT32", [3, 5, 64], 1),
    ("FLOAT16", [5, 4096], 0), ("INT8", [6, 4096], 0), ("UINT16", [4, 1000], 0), ("INT64", [8, 130], 0),
    ("FLOAT32", [13, 4096], 0), ("FLOAT32", [24, 520], 0), ("FLOAT16", [31, 96], 0), ("FLOAT32", [9, 3, 40], 0)])
@pytest.mark.parametrize("opn", OPS)
def test_plans_lane_short_and_tails(mx, orc, dt, shape, axis, opn):
    """Rows of <= 4 vectors (one lane per output), strided axes of <= 8 elements (all loads at
    once, 1 or 4 waves per block, 128-bit output stores) and strided axes of 9..31 elements
    (only the predicated tail of the four-wave columns plan runs)."""
    code, op = getattr(mx, dt), getattr(mx, opn)
    npt = mx.NP_DTYPE[code]
    rng = np.random.default_rng(7)
    xf = np.round(rng.standard_normal(shape) * 3)
    if code == mx.FLOAT32:
        x = xf.astype(np.float32)
        x[rng.random(shape) < 0.1] *= -0.0
    elif code == mx.FLOAT16:
        x = xf.astype(np.float16)
    elif code == mx.BFLOAT16:
        from oracle.oracle import f32_to_bf16_bits
        x = f32_to_bf16_bits(xf.astype(np.float32))
    else:
        info = np.iinfo(npt)
        x = rng.integers(info.min, info.max, size=shape, dtype=npt, endpoint=True)
    got, ref, *_ = run_reduce(mx, orc, op, code, x.ravel(), shape, axis)
    if op == mx.RED_SUM and code == mx.FLOAT32:
        check_sum(got, ref, abs_sum(mx, x.ravel(), shape, axis))
    else:
        # integer-valued 16-bit floats sum exactly in fp32, so both round the same exact sum
        assert np.array_equal(bits(got), bits(ref)), (dt, shape, axis, opn)


@pytest.mark.parametrize("dt", ["FLOAT32", "FLOAT16", "BFLOAT16", "INT32"])
@pytest.mark.parametrize("nv", [1, 2, 3, 4])
@pytest.mark.parametrize("opn", OPS)
def test_lane_plan_packed_and_gapped_rows(mx, orc, dt, nv, opn):
    """Rows of nv 16-byte vectors stored back to back (the block's rows are loaded as one run and
    staged in LDS) and the same rows with a one-vector gap after each (one lane loads its own row):
    both must give the oracle's bits, with a partial last block of rows."""
    code, op = getattr(mx, dt), getattr(mx, opn)
    vec = 16 // np.dtype(mx.NP_DTYPE[code]).itemsize
    n = nv * vec
    rng = np.random.default_rng(nv * 31 + code)
    for rows in (3, 256, 1000):
        xf = np.round(rng.standard_normal([rows, n + vec]) * 4).astype(np.float32)
        if code == mx.FLOAT16:
            xg = xf.astype(np.float16)
        elif code == mx.BFLOAT16:
            from oracle.oracle import f32_to_bf16_bits
            xg = f32_to_bf16_bits(xf)
        elif code == mx.INT32:
            xg = xf.astype(np.int32)
        else:
            xg = xf
        xp = np.ascontiguousarray(xg[:, :n])
        got_p, ref_p, *_ = run_reduce(mx, orc, op, code, xp.ravel(), [rows, n], 1)
        got_g, ref_g, *_ = run_reduce(mx, orc, op, code, xg.ravel(), [rows, n], 1, in_strides=[n + vec, 1])
        # integer-valued inputs: float sums are exact, so every op is bit-exact
        assert np.array_equal(bits(got_p), bits(ref_p)), (dt, nv, rows, opn, "packed")
        assert np.array_equal(bits(got_g), bits(ref_g)), (dt, nv, rows, opn, "gapped")
        assert np.array_equal(bits(got_p), bits(got_g)), (dt, nv, rows, opn)


@pytest.mark.parametrize("shape,axis", [([1, 5120], 1), ([5120], 0), ([512, 10], 0), ([2, 8192], 1), ([128, 128], 0)])
@pytest.mark.parametrize("opn", OPS)
def test_small_reductions_take_one_launch(mx, orc, shape, axis, opn):
    """At most 64 KiB of input: no split of the axis (no workspace, no combine launch), same
    results as the oracle (a loss, a bias gradient)."""
    op = getattr(mx, opn)
    rng = np.random.default_rng(sum(shape) + axis)
    x = np.round(rng.standard_normal(shape) * 4).astype(np.float32)
    desc, rs, n, total = reduce_desc(mx, shape, axis)
    assert mx.reduce_workspace_bytes(op, mx.FLOAT32, rs, n, desc) == 0
    got, ref, *_ = run_reduce(mx, orc, op, mx.FLOAT32, x.ravel(), shape, axis)
    assert np.array_equal(bits(got), bits(ref)), (shape, axis, opn)


@pytest.mark.parametrize("opn", OPS)
def test_unaligned_input_and_output(mx, orc, opn):
    """Views at a 4-byte offset: scalar loads for the lane / short plans, scalar output stores."""
    op = getattr(mx, opn)
    rng = np.random.default_rng(8)
    for shape, axis in [([600, 16], 1), ([600, 4], 1), ([6, 8192], 0), ([4, 4, 512], 1)]:
        x = np.round(rng.standard_normal(shape) * 3).astype(np.float32)
        desc, rs, n, total = reduce_desc(mx, shape, axis)
        X = mx.DeviceBuffer(x.nbytes + 16)
        X.upload(np.concatenate([np.zeros(1, np.float32), x.ravel()]).view(np.uint8))
        out_dt = np.int32 if op in (mx.RED_ARGMAX, mx.RED_ARGMIN) else np.float32
        O = mx.DeviceBuffer(total * 4 + 16)
        wsb = mx.reduce_workspace_bytes(op, mx.FLOAT32, rs, n, desc)
        W = mx.DeviceBuffer(wsb) if wsb else None
        mx.launch_reduce(op, mx.FLOAT32, rs, n, desc, O.ptr + 4, X.ptr + 4, W.ptr if W else 0, wsb)
        mx.sync()
        got = O.download(out_dt, total + 1)[1:]
        ref = orc.reduce(op, mx.FLOAT32, rs, n, desc, total, x.ravel(), acc=orc.ACC_F32)
        if op == mx.RED_SUM:
            check_sum(got, ref, abs_sum(mx, x.ravel(), shape, axis))
        else:
            assert np.array_equal(bits(got), bits(ref)), (shape, axis)
