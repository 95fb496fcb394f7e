"""Host shape helpers (matrix_amd/host/shape.cpp) against hand-derived collapse results.

Expected values are worked by hand from the merge rules of Mods/Utils.mm:114-435 and
Matrix.mm:161-331 at the workload shapes (add + row-sum, reductions, batched matmul).
"""
import pytest

import matrix_amd as mx
from helpers import contiguous_strides


def test_add_rowsum_add_collapse():
    # A[4096,1024] + B[1,1024]: B's 0 row stride blocks the merge -> 2 dims
    out, out_st, b1s, b1st, b2s, b2st = mx.broadcast_shapes([4096, 1024], [1024, 1], [1, 1024], [1024, 1])
    assert out == [4096, 1024] and out_st == [1024, 1]
    assert b1st == [1024, 1] and b2st == [0, 1]
    shape, sA, sB, sC = mx.collapse_dims3(b1s, b1st, b2st, out_st)
    assert (shape, sA, sB, sC) == ([4096, 1024], [1024, 1], [0, 1], [1024, 1])


def test_full_merge_when_all_contiguous():
    shape, sA, sB, sC = mx.collapse_dims3([8, 16, 32], [512, 32, 1], [512, 32, 1], [512, 32, 1])
    assert (shape, sA, sB, sC) == ([4096], [1], [1], [1])


def test_size_one_axes_dropped_but_not_axis0():
    shape, sA, sB, sC = mx.collapse_dims3([1, 5, 1, 3], [15, 3, 3, 1], [0, 0, 0, 1], [15, 3, 3, 1])
    # axis 0 (size 1) seeds the slot; axis 1 cannot merge (15 != 3*5 for B: 0 == 0*5 ok, A: 15==3*5 ok,
    # C: 15 == 3*5 ok) -> merges to [5]; axis 2 skipped; axis 3: A 3==1*3, B 0 != 1*3 -> new slot
    assert shape == [5, 3] and sA == [3, 1] and sB == [0, 1] and sC == [3, 1]


def test_rowsum_reduce_collapse():
    # sum(1) of [4096,1024], keepdims=False: out [4096] strides [1]
    shape, so, si = mx.collapse_dims_reduce2([4096, 1024], [1], [1024, 1], axis=1)
    assert (shape, so, si) == ([4096], [1], [1024])


@pytest.mark.parametrize("axis,exp", [
    (1, ([256], [1], [65536])),
    (0, ([65536], [1], [1])),
])
def test_reductions_256x65536(axis, exp):
    out_shape = [256, 65536][:axis] + [256, 65536][axis + 1:]
    got = mx.collapse_dims_reduce2([256, 65536], contiguous_strides(out_shape), [65536, 1], axis=axis)
    assert tuple(got) == exp


def test_reshaped_chain_sum3_then_sum1():
    # [64,4,4096,16].sum(3): everything merges into one slot of 1048576 with input stride 16
    got = mx.collapse_dims_reduce2([64, 4, 4096, 16], [16384, 4096, 1], [262144, 65536, 16, 1], axis=3)
    assert got == [[1048576], [1], [16]]
    # then .sum(1) on [64,4,4096] (contiguous): split at the axis -> [64,4096]
    got = mx.collapse_dims_reduce2([64, 4, 4096], [4096, 1], [16384, 4096, 1], axis=1)
    assert got == [[64, 4096], [4096, 1], [16384, 1]]


def test_keepdims_reduce():
    # keep_dims output strides, outer_collapsed=False (the reference passes !keepdims)
    got = mx.collapse_dims_reduce2([3, 1, 4], [4, 4, 1], [4, 4, 1], axis=1, keep_dims=False, outer_collapsed=False)
    assert got == [[3, 4], [4, 1], [4, 1]]


def test_matmul_collapse_batch_broadcast():
    # A[16,2048,2048] . Bt[2048,2048] -> batch stride of Bt is 0
    out, out_st, b1s, b1st, b2s, b2st = mx.broadcast_shapes([16, 2048, 2048], [2048 * 2048, 2048, 1],
                                                            [2048, 2048], [2048, 1], matmul=True)
    assert out == [16, 2048, 2048] and b2st == [0, 2048, 1]
    shape, sA, sB, sC = mx.collapse_dims_matmul(out, b1st, b2st, out_st)
    assert shape == [16, 2048, 2048]
    assert sA == [4194304, 2048, 1] and sB == [0, 2048, 1] and sC == [4194304, 2048, 1]


def test_matmul_collapse_skinny_and_4d():
    out, out_st, _, b1st, _, b2st = mx.broadcast_shapes([8, 1, 4096], [4096, 4096, 1], [4096, 4096], [4096, 1],
                                                        matmul=True)
    assert mx.collapse_dims_matmul(out, b1st, b2st, out_st) == [[8, 1, 4096], [4096, 4096, 1], [0, 4096, 1],
                                                                [4096, 4096, 1]]
    # two contiguous batch axes merge
    out, out_st, _, b1st, _, b2st = mx.broadcast_shapes([2, 3, 4, 5], contiguous_strides([2, 3, 4, 5]),
                                                        [2, 3, 6, 5], contiguous_strides([2, 3, 6, 5]), matmul=True)
    got = mx.collapse_dims_matmul(out, b1st, b2st, out_st)
    assert got[0] == [6, 4, 6] and got[1] == [20, 5, 1] and got[2] == [30, 5, 1] and got[3] == [24, 6, 1]


def test_broadcast_errors():
    with pytest.raises(mx.MatrixAMDError, match="Incompatible shapes"):
        mx.broadcast_shapes([3, 4], [4, 1], [5], [1])
    with pytest.raises(mx.MatrixAMDError, match="core dimension"):
        mx.broadcast_shapes([3, 4], [4, 1], [5, 5], [5, 1], matmul=True)
    with pytest.raises(mx.MatrixAMDError, match="enough dimensions"):
        mx.broadcast_shapes([4], [1], [5, 4], [4, 1], matmul=True)
