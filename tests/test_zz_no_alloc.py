"""GPU parity of mx_launch_reduce_noalloc, the allocation-free form of mx_launch_reduce: split
reductions whose partials go to the library's fixed per-GPU scratch instead of a caller workspace
must give mx_launch_reduce's outputs bit for bit, on consecutive calls of different sizes (the
second smaller, so it runs over the first call's leftover partials), without any device
allocation; a reduction needing more partials than the scratch holds is refused before any launch."""
import numpy as np
import pytest

from helpers import contiguous_strides

pytestmark = pytest.mark.gpu

OPS = ["RED_SUM", "RED_MAX", "RED_MIN", "RED_ARGMAX", "RED_ARGMIN"]


def plan(mx, shape, axis):
    out_shape = [s for i, s in enumerate(shape) if i != axis]
    desc = mx.collapse_dims_reduce2(shape, contiguous_strides(out_shape), contiguous_strides(shape), axis)
    return desc, contiguous_strides(shape)[axis], shape[axis], int(np.prod(out_shape))


def with_workspace(mx, op, x, shape, axis, out_dt):
    desc, rs, n, total = plan(mx, shape, axis)
    X = mx.DeviceBuffer.from_numpy(x)
    O = mx.DeviceBuffer(total * np.dtype(out_dt).itemsize)
    wsb = mx.reduce_workspace_bytes(op, mx.FLOAT32, rs, n, desc)
    W = mx.DeviceBuffer(wsb) if wsb else None
    mx.launch_reduce(op, mx.FLOAT32, rs, n, desc, O.ptr, X.ptr, W.ptr if W else 0, wsb)
    mx.sync()
    return O.download(out_dt, total), wsb


@pytest.mark.parametrize("opn", OPS)
@pytest.mark.parametrize("first,second", [
    (([512, 65280], 0), ([300, 20000], 0)),        # column plan split over blocks
    (([4, 1 << 20], 1), ([2, 300000], 1)),         # long rows split over blocks
    (([64, 256], 1), ([8, 100], 0)),               # no split at all: no scratch used
])
def test_noalloc_equals_workspace_form(mx, opn, first, second):
    op = getattr(mx, opn)
    out_dt = np.int32 if op in (mx.RED_ARGMAX, mx.RED_ARGMIN) else np.float32
    rng = np.random.default_rng(5)
    cases = []
    for shape, axis in (first, second):
        x = rng.standard_normal(shape).astype(np.float32)
        ref, wsb = with_workspace(mx, op, x.ravel(), shape, axis, out_dt)
        assert wsb <= mx.REDUCE_NOALLOC_SCRATCH_BYTES
        desc, rs, n, total = plan(mx, shape, axis)
        X = mx.DeviceBuffer.from_numpy(x.ravel())
        O = mx.DeviceBuffer(total * np.dtype(out_dt).itemsize)
        O.fill_bytes(0xA5)
        cases.append((desc, rs, n, total, X, O, ref))
    before = mx.alloc_stats()
    for desc, rs, n, total, X, O, _ in cases:      # the two calls in a row, second smaller
        mx.launch_reduce_noalloc(op, mx.FLOAT32, rs, n, desc, O.ptr, X.ptr)
    mx.sync()
    assert mx.alloc_stats() == before
    for desc, rs, n, total, X, O, ref in cases:
        got = O.download(out_dt, total)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (opn, first, second)


def test_noalloc_refuses_oversized_partials(mx):
    """uint8 Max over axis 0 of [512, 261120] needs 6,266,880 bytes of partials (above 4 MiB)."""
    shape, axis = [512, 261120], 0
    desc, rs, n, total = plan(mx, shape, axis)
    assert mx.reduce_workspace_bytes(mx.RED_MAX, mx.UINT8, rs, n, desc) > mx.REDUCE_NOALLOC_SCRATCH_BYTES
    X = mx.DeviceBuffer(512 * 261120)
    O = mx.DeviceBuffer(261120)
    with pytest.raises(mx.MatrixAMDError) as e:
        mx.launch_reduce_noalloc(mx.RED_MAX, mx.UINT8, rs, n, desc, O.ptr, X.ptr)
    assert e.value.status == mx.ERR_WORKSPACE and "4194304" in str(e.value)
