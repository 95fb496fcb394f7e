"""GPU parity: mx_launch_bcast_binary_reduce_rows (a broadcast op whose result is also reduced
over its rows).  R must equal mx_launch_bcast_binary's result bit for bit; the reduction must
equal the oracle's reduction of the oracle's R: bit-exact for Max / Min / ArgMax / ArgMin and
integer sums, |gpu - cpu| <= 1e-4 * sum|x| per row for fp32 sums, and the fp32-accumulate oracle
(one rounding) within 1e-3 relative for 16-bit sums of integer-valued data (exact partial sums)."""
import numpy as np
import pytest

from helpers import bits, contiguous_strides

pytestmark = pytest.mark.gpu

OPS = ["OP_ADD", "OP_SUB", "OP_MUL", "OP_DIV", "OP_MAX", "OP_MIN"]
REDS = ["RED_SUM", "RED_MAX", "RED_MIN", "RED_ARGMAX", "RED_ARGMIN"]


def make(rng, code, shape, mx):
    x = np.round(rng.standard_normal(shape) * 4).astype(np.float32) + 0.5
    if code == mx.FLOAT16:
        return x.astype(np.float16)
    if code == mx.BFLOAT16:
        from oracle.oracle import f32_to_bf16_bits
        return f32_to_bf16_bits(x)
    if code == mx.INT32:
        return np.round(x * 3).astype(np.int32)
    return x


def run(mx, orc, op, red, code, a_shape, b_shape, seed=0):
    rng = np.random.default_rng(seed)
    a = make(rng, code, a_shape, mx)
    b = make(rng, code, b_shape, mx)
    out, out_st, _, a_st, _, b_st = mx.broadcast_shapes(a_shape, contiguous_strides(a_shape), b_shape,
                                                        contiguous_strides(b_shape))
    desc = mx.collapse_dims3(out, a_st, b_st, out_st)
    total = int(np.prod(out)) if out else 1
    n = out[-1]
    A, B = mx.DeviceBuffer.from_numpy(a), mx.DeviceBuffer.from_numpy(b)
    R = mx.DeviceBuffer(total * a.itemsize)
    R2 = mx.DeviceBuffer(total * a.itemsize)
    o_dt = np.int32 if red in (mx.RED_ARGMAX, mx.RED_ARGMIN) else a.dtype
    O = mx.DeviceBuffer(total // n * np.dtype(o_dt).itemsize)
    mx.launch_bcast_binary_reduce_rows(op, red, code, desc, n, R.ptr, A.ptr, B.ptr, O.ptr)
    mx.launch_bcast_binary(op, code, desc, R2.ptr, A.ptr, B.ptr)
    mx.sync()
    r_got, r_unfused = R.download(a.dtype, total), R2.download(a.dtype, total)
    assert np.array_equal(bits(r_got), bits(r_unfused)), "R differs from the broadcast kernel"
    r_ref = orc.bcast_binary(op, code, desc, total, a.ravel(), b.ravel())
    assert np.array_equal(bits(r_got), bits(r_ref)), "R differs from the oracle"
    rdesc = [[total // n], [1], [n]]
    ref = orc.reduce(red, code, 1, n, rdesc, total // n, r_ref, acc=orc.ACC_F32)
    got = O.download(o_dt, total // n)
    return got, ref, r_ref.reshape(-1, n)


def as_f32(code, x, mx):
    if code == mx.BFLOAT16:
        return (x.astype(np.uint32) << 16).view(np.float32)
    return x.astype(np.float32)


@pytest.mark.parametrize("red", REDS)
@pytest.mark.parametrize("op", OPS)
def test_add_rowsum_shape_every_op(mx, orc, op, red):
    """Config 1's shape A[4096,1024] op B[1,1024], float32, every op and reduction."""
    o, r = getattr(mx, op), getattr(mx, red)
    got, ref, rows = run(mx, orc, o, r, mx.FLOAT32, [4096, 1024], [1, 1024])
    if r == mx.RED_SUM:
        mag = np.abs(rows.astype(np.float64)).sum(1)
        assert np.all(np.abs(got.astype(np.float64) - ref) <= 1e-4 * mag + 1e-30)
    else:
        assert np.array_equal(bits(got), bits(ref))


@pytest.mark.parametrize("dt", ["FLOAT32", "FLOAT16", "BFLOAT16", "INT32"])
@pytest.mark.parametrize("shapes", [
    ([64, 96], [64, 1]),            # B broadcast along the row (stride 0 inner axis)
    ([33, 40], []),                 # scalar B
    ([5, 7, 24], [7, 24]),          # three axes, B broadcast over the first
    ([16, 4096], [1, 4096]),        # 16 KiB rows (fp32)
    ([10, 13], [10, 13]),           # rows not a whole number of vectors: two kernels
    ([6, 8], [1, 8]),               # tiny
])
@pytest.mark.parametrize("red", ["RED_SUM", "RED_MAX", "RED_ARGMIN"])
def test_dtypes_and_layouts(mx, orc, dt, shapes, red):
    code, r = getattr(mx, dt), getattr(mx, red)
    a_shape, b_shape = shapes
    got, ref, rows = run(mx, orc, mx.OP_ADD, r, code, a_shape, b_shape, seed=3)
    if r == mx.RED_SUM and code == mx.FLOAT32:
        mag = np.abs(rows.astype(np.float64)).sum(1)
        assert np.all(np.abs(got.astype(np.float64) - ref) <= 1e-4 * mag + 1e-30)
    elif r == mx.RED_SUM and code in (mx.FLOAT16, mx.BFLOAT16):
        g, w = as_f32(code, got, mx), as_f32(code, ref, mx)
        assert np.all(np.abs(g - w) <= 1e-3 * np.maximum(np.abs(w), 1.0))
    else:
        assert np.array_equal(bits(got), bits(ref))


def test_rows_above_16k_rejected(mx):
    desc = ([2, 8192], [8192, 1], [8192, 1], [8192, 1])
    X = mx.DeviceBuffer(2 * 8192 * 4)
    O = mx.DeviceBuffer(16)
    with pytest.raises(mx.MatrixAMDError, match="16 KiB"):
        mx.launch_bcast_binary_reduce_rows(mx.OP_ADD, mx.RED_SUM, mx.FLOAT32, desc, 8192, X.ptr, X.ptr, X.ptr, O.ptr)
    with pytest.raises(mx.MatrixAMDError, match="divide"):
        mx.launch_bcast_binary_reduce_rows(mx.OP_ADD, mx.RED_SUM, mx.FLOAT32, desc, 3000, X.ptr, X.ptr, X.ptr, O.ptr)
