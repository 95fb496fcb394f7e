"""GPU parity: mx_launch_max_grad -- the gradient Max / Min send to one operand, in one launch.

The vjp of Max / Min (primitives.cpp:2604-2608) is four broadcast launches: m = max|min(a, b),
mask_b = equal(b, m), then g * (1 - mask_b) for a and g * mask_b for b.  The fused launch must give
their result bit for bit: ties (a == b, including +0 / -0) send g to b, NaN operands follow the
select, and g * 0 keeps g's sign (-0 for negative g).  Shapes cover the ReLU of a dense layer
(b a scalar), a bias row, ragged broadcasts on the one-element path and rank 0.  The fused launch
is also checked against the same four steps run in the oracle.
"""
import numpy as np
import pytest

from helpers import bits, contiguous_strides

pytestmark = pytest.mark.gpu


def stored(mx, code, x):
    x = np.asarray(x, np.float32)
    if code == mx.FLOAT16:
        return x.astype(np.float16)
    if code == mx.BFLOAT16:
        from oracle.oracle import f32_to_bf16_bits
        return f32_to_bf16_bits(x)
    return x


def desc(mx, sx, sy):
    out, out_st, b1s, b1st, b2s, b2st = mx.broadcast_shapes(list(sx), contiguous_strides(list(sx)), list(sy),
                                                            contiguous_strides(list(sy)))
    if not out:
        return [], [], [], [], out
    return (*mx.collapse_dims3(b1s, b1st, b2st, out_st), out)


def values(rng, shape, special):
    x = np.round(rng.standard_normal(shape) * 2).astype(np.float32)   # many exact ties and zeros
    if special and x.size >= 16:
        flat = x.reshape(-1)
        flat[:8] = [np.nan, -0.0, 0.0, np.inf, -np.inf, -0.0, 1.0, np.nan]
    return x


def run_case(mx, code, op, sa, sb, seed, special=True, orc=None):
    rng = np.random.default_rng(seed)
    npt = mx.NP_DTYPE[code]
    a = stored(mx, code, values(rng, sa, special))
    b = stored(mx, code, values(rng, sb, special))
    out_shape = list(np.broadcast_shapes(tuple(sa), tuple(sb)))
    g = stored(mx, code, rng.standard_normal(out_shape).astype(np.float32))   # negative g: g * 0 = -0
    total = int(np.prod(out_shape)) if out_shape else 1
    esz = np.dtype(npt).itemsize
    A, B, G = (mx.DeviceBuffer.from_numpy(np.ascontiguousarray(v).reshape(-1)) for v in (a, b, g))
    one = mx.DeviceBuffer.from_numpy(stored(mx, code, [1.0]))
    buf = lambda: mx.DeviceBuffer(max(total, 1) * esz)
    # the four launches of the vjp
    M, MB, MA, RA, RB = buf(), buf(), buf(), buf(), buf()
    d_ab = desc(mx, sa, sb)[:4]
    d_full = desc(mx, out_shape, out_shape)[:4]
    d_one = desc(mx, [], out_shape)[:4]
    d_b_full = desc(mx, sb, out_shape)[:4]
    mx.launch_bcast_binary(op, code, d_ab, M.ptr, A.ptr, B.ptr)
    mx.launch_bcast_binary(mx.OP_EQ, code, d_b_full, MB.ptr, B.ptr, M.ptr)
    mx.launch_bcast_binary(mx.OP_SUB, code, d_one, MA.ptr, one.ptr, MB.ptr)
    mx.launch_bcast_binary(mx.OP_MUL, code, d_full, RA.ptr, G.ptr, MA.ptr)
    mx.launch_bcast_binary(mx.OP_MUL, code, d_full, RB.ptr, G.ptr, MB.ptr)
    # the fused launches
    FA, FB = buf(), buf()
    for F in (FA, FB):
        F.fill_bytes(0xA5)
    mx.launch_max_grad(op, 0, code, d_ab, FA.ptr, A.ptr, B.ptr, G.ptr)
    mx.launch_max_grad(op, 1, code, d_ab, FB.ptr, A.ptr, B.ptr, G.ptr)
    mx.sync()
    for side, (F, R) in enumerate([(FA, RA), (FB, RB)]):
        got, ref = F.download(npt, total), R.download(npt, total)
        assert np.array_equal(bits(got), bits(ref)), (code, op, sa, sb, side)
    if orc is not None:
        # the same four steps in the oracle (the reference's CPU loops), against the fused launch
        flat = lambda v: np.ascontiguousarray(v).reshape(-1)
        m = orc.bcast_binary(op, code, d_ab, total, flat(a), flat(b))
        mb = orc.bcast_binary(orc.EQ, code, d_b_full, total, flat(b), m)
        ma = orc.bcast_binary(orc.SUB, code, d_one, total, flat(stored(mx, code, [1.0])), mb)
        for side, (F, mask) in enumerate([(FA, ma), (FB, mb)]):
            want = orc.bcast_binary(orc.MUL, code, d_full, total, flat(g), mask)
            assert np.array_equal(bits(F.download(npt, total)), bits(want)), ("oracle", code, op, sa, sb, side)
    return FA.download(npt, total), FB.download(npt, total)


@pytest.mark.parametrize("dt", ["FLOAT32", "FLOAT16", "BFLOAT16"])
@pytest.mark.parametrize("opn", ["OP_MAX", "OP_MIN"])
@pytest.mark.parametrize("sa,sb", [
    ([512, 4096], []),              # ReLU of a dense layer: b the scalar 0 (here random)
    ([64, 96], [96]),               # a bias row
    ([7, 5, 3], [7, 1, 1]),         # ragged: one element per thread
    ([1, 5, 3], [7, 1, 3]),         # both broadcast
    ([], []),                       # rank 0
])
def test_max_grad_equals_four_launches(mx, orc, dt, opn, sa, sb):
    run_case(mx, getattr(mx, dt), getattr(mx, opn), sa, sb, seed=len(sa) * 10 + len(sb), orc=orc)


def test_max_grad_routes_ties_to_b(mx):
    """Where a == b the whole gradient goes to b (a gets +-0); elsewhere to the larger operand."""
    code = mx.FLOAT32
    ga, gb = run_case(mx, code, mx.OP_MAX, [4096], [], seed=3, special=False)
    rng = np.random.default_rng(3)                  # the same inputs again on the host
    a = values(rng, [4096], False)
    b = float(values(rng, [], False))
    g = rng.standard_normal([4096]).astype(np.float32)
    ties = a == b
    assert ties.any() and (a > b).any() and (a < b).any()
    to_b = a <= b
    assert np.array_equal(gb[to_b], g[to_b]) and np.all(ga[to_b] == 0)
    assert np.array_equal(ga[~to_b], g[~to_b]) and np.all(gb[~to_b] == 0)


def test_max_grad_errors(mx):
    X = mx.DeviceBuffer(64)
    d = desc(mx, [4], [4])[:4]
    with pytest.raises(mx.MatrixAMDError):
        mx.launch_max_grad(mx.OP_ADD, 0, mx.FLOAT32, d, X.ptr, X.ptr, X.ptr, X.ptr)
    with pytest.raises(mx.MatrixAMDError):
        mx.launch_max_grad(mx.OP_MAX, 2, mx.FLOAT32, d, X.ptr, X.ptr, X.ptr, X.ptr)
    with pytest.raises(mx.MatrixAMDError) as e:
        mx.launch_max_grad(mx.OP_MAX, 0, mx.INT32, d, X.ptr, X.ptr, X.ptr, X.ptr)
    assert e.value.status == mx.ERR_UNSUPPORTED
