"""GPU parity: mx_launch_reduce_group -- several reductions over one descriptor in one launch.

Each member runs the plan body of its own single-op kernel, so its output must equal that of
mx_launch_reduce bit for bit, and through it the oracle (Max / Min / ArgMax / ArgMin and integer
sums bit-exact; float sums of integer-valued inputs exact, of N(0, 1) inputs within
1e-4 * sum|x| per output).  Every member reads its own input, so a member reading or writing
another's buffers shows.  The shapes cover each plan: lane (rows of <= 4 vectors), rows, block
(long rows, with and without a split axis), short (strided, <= 8 elements) and cols (strided,
with and without a split axis).  INT32 takes the per-member fallback.
"""
import numpy as np
import pytest

from helpers import bits, contiguous_strides
from test_gpu_reduce import abs_sum, check_sum, reduce_desc

pytestmark = pytest.mark.gpu

ALL_OPS = ["RED_SUM", "RED_MAX", "RED_MIN", "RED_ARGMAX", "RED_ARGMIN"]

PLAN_CASES = [
    ([4096, 16], 1),          # lane: rows of 4 vectors (f32)
    ([1000, 16], 1),          # lane with a partial last block
    ([777, 32], 1),           # lane for 16-bit types (4 vectors), rows for 32-bit
    ([500, 12], 1),           # lane: 3 vectors
    ([1000, 200], 1),         # rows: 50 vectors per row
    ([256, 32768], 1),        # block, 16 waves, one block per output
    ([16, 65536], 1),         # block, axis split over blocks (16 outputs), combine launch
    ([16, 4, 1024, 16], 1),   # short: n = 4, stride 16384
    ([40, 65536], 0),         # cols, no split
    ([300, 2000], 0),         # cols, axis split (8 column groups)
]


def storage(mx, code, xf):
    if code == mx.FLOAT16:
        return xf.astype(np.float16)
    if code == mx.BFLOAT16:
        from oracle.oracle import f32_to_bf16_bits
        return f32_to_bf16_bits(xf)
    if code == mx.INT32:
        return xf.astype(np.int32)
    return xf.astype(np.float32)


def run_group(mx, orc, code, ops, xs, shape, axis):
    """Group launch, then each member alone; returns [(group out, single out, oracle)]."""
    desc, rs, n, total = reduce_desc(mx, shape, axis)
    outs, singles, ins, wss, wsbs, keep = [], [], [], [], [], []
    for op, x in zip(ops, xs):
        X = mx.DeviceBuffer.from_numpy(x.ravel())
        out_dt = np.int32 if op in (mx.RED_ARGMAX, mx.RED_ARGMIN) else x.dtype
        O = mx.DeviceBuffer(total * np.dtype(out_dt).itemsize)
        O.fill_bytes(0xA5)
        wsb = mx.reduce_workspace_bytes(op, code, rs, n, desc)
        W = mx.DeviceBuffer(wsb) if wsb else None
        keep += [X, O, W]
        ins.append(X.ptr)
        outs.append((O, out_dt))
        wss.append(W.ptr if W else 0)
        wsbs.append(wsb)
    mx.launch_reduce_group(ops, code, rs, n, desc, [o.ptr for o, _ in outs], ins, wss, wsbs)
    mx.sync()
    got = [o.download(dt, total) for o, dt in outs]
    for k, op in enumerate(ops):
        S = mx.DeviceBuffer(total * np.dtype(outs[k][1]).itemsize)
        mx.launch_reduce(op, code, rs, n, desc, S.ptr, ins[k], wss[k], wsbs[k])
        mx.sync()
        singles.append(S.download(outs[k][1], total))
    refs = [orc.reduce(op, code, rs, n, desc, total, x.ravel(), acc=orc.ACC_F32) for op, x in zip(ops, xs)]
    return list(zip(got, singles, refs))


@pytest.mark.parametrize("dt", ["FLOAT32", "FLOAT16", "BFLOAT16", "INT32"])
@pytest.mark.parametrize("shape,axis", PLAN_CASES)
def test_group_of_all_ops_matches_single_launches(mx, orc, dt, shape, axis):
    code = getattr(mx, dt)
    ops = [getattr(mx, o) for o in ALL_OPS]
    rng = np.random.default_rng(sum(shape) * 7 + axis)
    # integer-valued inputs: many ties for the arg reductions, and exact float sums
    xs = [storage(mx, code, np.round(rng.standard_normal(shape) * 8).astype(np.float32)) for _ in ops]
    for k, (g, s, r) in enumerate(run_group(mx, orc, code, ops, xs, shape, axis)):
        assert np.array_equal(bits(g), bits(s)), (dt, shape, axis, ALL_OPS[k], "group != single launch")
        assert np.array_equal(bits(g), bits(r)), (dt, shape, axis, ALL_OPS[k], "group != oracle")


@pytest.mark.parametrize("shape,axis", [([256, 32768], 1), ([16, 4, 1024, 16], 3), ([300, 2000], 0)])
def test_group_f32_sums_and_ties(mx, orc, shape, axis):
    """N(0, 1) inputs with injected duplicate extrema; members in a different order and count."""
    from test_gpu_reduce import inject_ties
    code = mx.FLOAT32
    names = ["RED_ARGMIN", "RED_SUM", "RED_ARGMAX"]
    ops = [getattr(mx, o) for o in names]
    rng = np.random.default_rng(3)
    xs = [inject_ties(rng, rng.standard_normal(shape).astype(np.float32), axis, minimum=(o == "RED_ARGMIN"))
          for o in names]
    for k, (g, s, r) in enumerate(run_group(mx, orc, code, ops, xs, shape, axis)):
        assert np.array_equal(bits(g), bits(s)), (shape, axis, names[k])
        if names[k] == "RED_SUM":
            check_sum(g, r, abs_sum(mx, xs[k].ravel(), shape, axis))
        else:
            assert np.array_equal(g, r), (shape, axis, names[k])


def test_group_errors_and_edge_sizes(mx, orc):
    code = mx.FLOAT32
    desc, rs, n, total = reduce_desc(mx, [16, 65536], 1)
    X = mx.DeviceBuffer.from_numpy(np.ones(16 * 65536, np.float32))
    O = [mx.DeviceBuffer(16 * 4) for _ in range(2)]
    # the split plan needs each member's workspace
    with pytest.raises(mx.MatrixAMDError) as e:
        mx.launch_reduce_group([mx.RED_SUM, mx.RED_MAX], code, rs, n, desc, [O[0].ptr, O[1].ptr], [X.ptr, X.ptr])
    assert e.value.status == mx.ERR_WORKSPACE
    with pytest.raises(mx.MatrixAMDError):
        mx.launch_reduce_group([mx.RED_SUM] * 9, code, rs, n, desc, [O[0].ptr] * 9, [X.ptr] * 9)
    mx.launch_reduce_group([], code, rs, n, desc, [], [])           # nothing to do
    # one member equals mx_launch_reduce
    wsb = mx.reduce_workspace_bytes(mx.RED_SUM, code, rs, n, desc)
    W = mx.DeviceBuffer(wsb)
    mx.launch_reduce_group([mx.RED_SUM], code, rs, n, desc, [O[0].ptr], [X.ptr], [W.ptr], [wsb])
    mx.sync()
    assert np.array_equal(O[0].download(np.float32, 16), np.full(16, 65536.0, np.float32))
