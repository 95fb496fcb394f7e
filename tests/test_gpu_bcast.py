"""GPU parity: broadcast binary kernels vs the oracle, bit-exact (divide: <= 1 ulp).

Descriptors come from the product's own broadcast + collapse helpers, exactly as the graph
layer builds them; the oracle runs the reference's CPU loop on the same descriptor.
"""
import numpy as np
import pytest

from helpers import bits, contiguous_strides

pytestmark = pytest.mark.gpu

DTYPES = ["FLOAT32", "FLOAT16", "BFLOAT16", "INT32", "INT8", "INT16", "INT64", "UINT8", "UINT16", "UINT32",
          "UINT64", "BOOL"]
OPS = ["OP_ADD", "OP_SUB", "OP_MUL", "OP_DIV", "OP_MAX", "OP_MIN", "OP_EQ"]


def make_data(rng, code, shape, mx, for_div=False):
    npt = mx.NP_DTYPE[code]
    if code in (mx.FLOAT32, mx.FLOAT16):
        x = rng.standard_normal(shape) * 4
        x = np.where(rng.random(shape) < 0.05, 0.0, x)       # exact ties / zeros
        return x.astype(npt)
    if code == mx.BFLOAT16:
        from oracle.oracle import f32_to_bf16_bits
        return f32_to_bf16_bits((rng.standard_normal(shape) * 4).astype(np.float32))
    if code == mx.BOOL:
        return rng.integers(0, 2, size=shape).astype(np.bool_)
    info = np.iinfo(npt)
    lo, hi = (info.min, info.max) if not for_div else (max(info.min, -1000), min(info.max, 1000))
    return rng.integers(lo, hi, size=shape, dtype=npt, endpoint=True)


def run_pair(mx, orc, op, code, a, b, a_strides=None, b_strides=None, a_shape=None, b_shape=None, offset_elems=0):
    a_shape = list(a_shape or a.shape)
    b_shape = list(b_shape or b.shape)
    a_strides = a_strides or contiguous_strides(a_shape)
    b_strides = b_strides or contiguous_strides(b_shape)
    out, out_st, b1s, b1st, b2s, b2st = mx.broadcast_shapes(a_shape, a_strides, b_shape, b_strides)
    if len(out):
        desc = mx.collapse_dims3(b1s, b1st, b2st, out_st)
    else:
        desc = [[], [], [], []]
    total = int(np.prod(out)) if out else 1
    esz = a.dtype.itemsize
    A = mx.DeviceBuffer(a.nbytes + offset_elems * esz + 16)
    B = mx.DeviceBuffer(b.nbytes + 16)
    R = mx.DeviceBuffer(max(total * esz, 1) + 16)
    A.upload(a.reshape(-1).view(np.uint8), offset_elems * esz)
    B.upload(b.reshape(-1).view(np.uint8))
    shape, sA, sB, sR = desc
    mx.launch_bcast_binary(op, code, (shape, sA, sB, sR), R.ptr, A.ptr + offset_elems * esz, B.ptr)
    mx.sync()
    got = R.download(a.dtype, total)
    ref = orc.bcast_binary(op, code, (shape, sA, sB, sR), total, a.reshape(-1), b.reshape(-1))
    return got, ref


def as_f32(code, arr, mx):
    if code == mx.BFLOAT16:
        return (arr.astype(np.uint32) << 16).view(np.float32)
    return arr.astype(np.float32)


def assert_match(got, ref, op, code, mx):
    """Bit-exact, except: a NaN produced by an invalid operation (0/0, inf-inf) matches any NaN,
    since the default NaN's sign differs between the oracle's x86 host (negative) and
    arm64 / gfx950 (positive); divide may differ by <= 1 ulp."""
    gi = bits(got).astype(np.int64)
    ri = bits(ref).astype(np.int64)
    if code in (mx.FLOAT32, mx.FLOAT16, mx.BFLOAT16):
        both_nan = np.isnan(as_f32(code, got, mx)) & np.isnan(as_f32(code, ref, mx))
    else:
        both_nan = np.zeros(got.shape, bool)
    tol = 1 if (op == mx.OP_DIV and code in (mx.FLOAT32, mx.FLOAT16, mx.BFLOAT16)) else 0
    bad = (np.abs(gi - ri) > tol) & ~both_nan
    assert not bad.any(), f"op {op} dtype {code}: {int(bad.sum())} mismatches, first at {int(np.argmax(bad))}"


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("opn", OPS)
def test_all_ops_all_dtypes(mx, orc, dt, opn):
    code, op = getattr(mx, dt), getattr(mx, opn)
    rng = np.random.default_rng(100 + code * 7 + op)
    for sa, sb in [([64, 96], [1, 96]), ([5, 7, 3], [7, 1]), ([33], [33]), ([8, 1], [1, 40])]:
        a = make_data(rng, code, sa, mx, op == mx.OP_DIV)
        b = make_data(rng, code, sb, mx, op == mx.OP_DIV)
        got, ref = run_pair(mx, orc, op, code, a, b)
        assert_match(got, ref, op, code, mx)


@pytest.mark.parametrize("opn", OPS)
def test_add_rowsum_shape_f32(mx, orc, opn):
    """A[4096,1024] ~ N(0,1) op B[1,1024] ~ U(-1,1), seed 0 (the add + row-sum workload)."""
    op = getattr(mx, opn)
    rng = np.random.default_rng(0)
    a = rng.standard_normal([4096, 1024]).astype(np.float32)
    b = rng.uniform(-1, 1, [1, 1024]).astype(np.float32)
    got, ref = run_pair(mx, orc, op, mx.FLOAT32, a, b)
    assert_match(got, ref, op, mx.FLOAT32, mx)


def test_special_float_values(mx, orc):
    nan, inf = np.nan, np.inf
    vals = np.array([0.0, -0.0, 1.0, -1.0, nan, inf, -inf, 1e-45, -1e-45, 3.4e38, -3.4e38, 2.5], np.float32)
    a = np.repeat(vals, len(vals))
    b = np.tile(vals, len(vals))
    for opn in OPS:
        op = getattr(mx, opn)
        got, ref = run_pair(mx, orc, op, mx.FLOAT32, a, b)
        assert_match(got, ref, op, mx.FLOAT32, mx)
        ah, bh = a.astype(np.float16), b.astype(np.float16)
        got, ref = run_pair(mx, orc, op, mx.FLOAT16, ah, bh)
        assert_match(got, ref, op, mx.FLOAT16, mx)


def test_integer_division_edges(mx, orc):
    for dt, npt in [("INT32", np.int32), ("INT8", np.int8), ("INT64", np.int64), ("UINT32", np.uint32)]:
        info = np.iinfo(npt)
        vals = [info.min, -7, -1, 0, 1, 7, info.max] if info.min < 0 else [0, 1, 7, info.max]
        a = np.array([x for x in vals for _ in vals], npt)
        b = np.array([y for _ in vals for y in vals], npt)
        code = getattr(mx, dt)
        got, ref = run_pair(mx, orc, mx.OP_DIV, code, a, b)
        assert np.array_equal(got, ref), dt


def test_scalar_paths_and_misaligned(mx, orc):
    rng = np.random.default_rng(7)
    # rank-0 op rank-0
    a = np.array(3.25, np.float32)
    b = np.array(-2.0, np.float32)
    got, ref = run_pair(mx, orc, mx.OP_MUL, mx.FLOAT32, a, b, a_shape=[], b_shape=[])
    assert_match(got, ref, mx.OP_MUL, mx.FLOAT32, mx)
    # matrix op rank-0 scalar (the MLP's ReLU max(x, 0))
    x = rng.standard_normal([512, 64]).astype(np.float32)
    z = np.array(0.0, np.float32)
    got, ref = run_pair(mx, orc, mx.OP_MAX, mx.FLOAT32, x, z, b_shape=[])
    assert np.array_equal(bits(got), bits(ref))
    # misaligned A base (one element off) forces the scalar kernel
    got, ref = run_pair(mx, orc, mx.OP_ADD, mx.FLOAT32, x, x[:1], offset_elems=1)
    assert np.array_equal(bits(got), bits(ref))
    # odd inner extent
    y = rng.standard_normal([37, 13]).astype(np.float32)
    got, ref = run_pair(mx, orc, mx.OP_SUB, mx.FLOAT32, y, y[:1])
    assert np.array_equal(bits(got), bits(ref))


def test_strided_view_operand(mx, orc):
    """A is a transposed view (strides [1, 48]) of a [48, 40] buffer."""
    rng = np.random.default_rng(8)
    base = rng.standard_normal([48, 40]).astype(np.float32)
    b = rng.standard_normal([40, 48]).astype(np.float32)
    got, ref = run_pair(mx, orc, mx.OP_ADD, mx.FLOAT32, base, b, a_shape=[40, 48], a_strides=[1, 40])
    assert np.array_equal(bits(got), bits(ref))
    assert np.array_equal(got.reshape(40, 48), base.T + b)


def complex_data(rng, shape):
    z = rng.standard_normal(list(shape) + [2]).astype(np.float32) * 4
    z[rng.random(shape) < 0.05] = 0.0                                   # zeros in both parts
    return z.view(np.complex64).reshape(shape)


def assert_complex_match(got, ref):
    """Bit-exact per part; a NaN part matches any NaN (0 / 0 from a zero divisor)."""
    g, r = got.view(np.float32), ref.view(np.float32)
    bad = (bits(g) != bits(r)) & ~(np.isnan(g) & np.isnan(r))
    assert not bad.any(), f"{int(bad.sum())} mismatching float parts, first at {int(np.argmax(bad))}"


@pytest.mark.parametrize("opn", ["OP_ADD", "OP_SUB", "OP_MUL", "OP_DIV"])
def test_complex64_ops(mx, orc, opn):
    """complex64 Add / Sub / Mul / Divide (complex.h:28-52) on the 16-byte path (even inner
    extent), the gather path (odd inner extent, row broadcast), rank-0 and a misaligned view."""
    op = getattr(mx, opn)
    rng = np.random.default_rng(300 + op)
    for sa, sb in [([64, 96], [1, 96]), ([5, 7, 3], [7, 1]), ([33], [33]), ([8, 1], [1, 40]), ([256, 1024], [1024])]:
        a, b = complex_data(rng, sa), complex_data(rng, sb)
        got, ref = run_pair(mx, orc, op, mx.COMPLEX64, a, b)
        assert_complex_match(got, ref)
    a, b = complex_data(rng, []), complex_data(rng, [])
    got, ref = run_pair(mx, orc, op, mx.COMPLEX64, a, b, a_shape=[], b_shape=[])
    assert_complex_match(got, ref)
    a, b = complex_data(rng, [48, 32]), complex_data(rng, [48, 32])
    got, ref = run_pair(mx, orc, op, mx.COMPLEX64, a, b, offset_elems=1)
    assert_complex_match(got, ref)


def test_complex64_has_no_ordering_ops(mx):
    A = mx.DeviceBuffer(64)
    for op in (mx.OP_MAX, mx.OP_MIN, mx.OP_EQ):
        with pytest.raises(mx.MatrixAMDError):
            mx.launch_bcast_binary(op, mx.COMPLEX64, ([4], [1], [1], [1]), A.ptr, A.ptr, A.ptr)
