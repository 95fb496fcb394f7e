"""Committed golden fixtures (tests/golden/golden.npz, written by tests/golden/make_golden.py from
numpy: IEEE float32 element-wise results, float64 sums / products / convolutions, numpy's
first-index argmax / argmin, in-range casts) checked against the oracle on the CPU and against
the kernels on the GPU."""
from pathlib import Path

import numpy as np
import pytest

from helpers import bcast_desc_uncollapsed, bits, contiguous_strides, normwise_rel

G = np.load(Path(__file__).resolve().parent / "golden" / "golden.npz")
OPS = ["add", "sub", "mul", "div", "max", "min", "eq"]


def red_desc(shape, axis):
    out_shape = [s for i, s in enumerate(shape) if i != axis]
    ins = contiguous_strides(shape)
    return (out_shape, contiguous_strides(out_shape), [s for i, s in enumerate(ins) if i != axis]), ins[axis], shape[axis]


# ------------------------------------------------------------------ oracle (CPU)
@pytest.mark.parametrize("i,name", list(enumerate(OPS)))
def test_oracle_bcast_golden(orc, i, name):
    a, b = G["bcast_a"], G["bcast_b"]
    desc = bcast_desc_uncollapsed(a.shape, b.shape)
    got = orc.bcast_binary(i, orc.F32, desc, a.size, a.ravel(), b.ravel())
    assert np.array_equal(bits(got), bits(G[f"bcast_{name}"].ravel()))


@pytest.mark.parametrize("axis", [0, 1])
def test_oracle_reduce_golden(orc, axis):
    x = G["red_x"]
    desc, rs, n = red_desc(list(x.shape), axis)
    total = int(np.prod(desc[0]))
    s = orc.reduce(orc.RSUM, orc.F32, rs, n, desc, total, x.ravel())
    assert np.all(np.abs(s - G[f"red_sum{axis}"]) <= 1e-6 * G[f"red_abs{axis}"])
    for op, key in ((orc.RMAX, "max"), (orc.RMIN, "min"), (orc.RARGMAX, "argmax"), (orc.RARGMIN, "argmin")):
        got = orc.reduce(op, orc.F32, rs, n, desc, total, x.ravel())
        assert np.array_equal(got, G[f"red_{key}{axis}"]), key


def test_oracle_matmul_conv_copy_golden(orc):
    a, b = G["mm_a"], G["mm_b"]
    bt = np.ascontiguousarray(b.T)
    desc = ([2, 9, 11], [9 * 13, 13, 1], [0, 13, 1], [9 * 11, 11, 1])
    c = orc.batched_matmul(orc.F32, desc, 13, a.ravel(), bt.ravel(), 2 * 9 * 11)
    assert normwise_rel(c, G["mm_c"]) <= 1e-6
    ci, ck = G["conv_in"], G["conv_k"]
    out = orc.conv(orc.F32, [2, 6, 5, 3], [4, 3, 3, 3], [2, 6, 5, 4], contiguous_strides([2, 6, 5, 3]),
                   contiguous_strides([4, 3, 3, 3]), contiguous_strides([2, 6, 5, 4]), [1, 1], [1, 1], [1, 1], [1, 1],
                   1, 0, ci.ravel(), ck.ravel(), 2 * 6 * 5 * 4)
    assert normwise_rel(out, G["conv_out"]) <= 1e-6
    src = G["cast_src"]
    i32 = orc.copy_strided(orc.I32, orc.F32, [40], [1], [1], np.zeros(40, np.int32), src)
    assert np.array_equal(i32, G["cast_i32"])
    f16 = orc.copy_strided(orc.F16, orc.F32, [40], [1], [1], np.zeros(40, np.uint16), src)
    assert np.array_equal(f16, G["cast_f16"])
    u8 = orc.copy_strided(orc.U8, orc.F32, [40], [1], [1], np.zeros(40, np.uint8), G["cast_u8_src"])
    assert np.array_equal(u8, G["cast_u8"])


# ------------------------------------------------------------------ kernels (GPU)
@pytest.mark.gpu
def test_kernels_golden(mx):
    a, b = G["bcast_a"], G["bcast_b"]
    desc = bcast_desc_uncollapsed(a.shape, b.shape)
    A, B = mx.DeviceBuffer.from_numpy(a), mx.DeviceBuffer.from_numpy(b)
    R = mx.DeviceBuffer(a.nbytes)
    for i, name in enumerate(OPS):
        mx.launch_bcast_binary(i, mx.FLOAT32, desc, R.ptr, A.ptr, B.ptr)
        mx.sync()
        assert np.array_equal(bits(R.download(np.float32)), bits(G[f"bcast_{name}"].ravel())), name

    x = G["red_x"]
    X = mx.DeviceBuffer.from_numpy(x)
    for axis in (0, 1):
        desc, rs, n = red_desc(list(x.shape), axis)
        total = int(np.prod(desc[0]))
        O = mx.DeviceBuffer(total * 4)
        for op, key in ((mx.RED_SUM, "sum"), (mx.RED_MAX, "max"), (mx.RED_MIN, "min"),
                        (mx.RED_ARGMAX, "argmax"), (mx.RED_ARGMIN, "argmin")):
            ws = mx.reduce_workspace_bytes(op, mx.FLOAT32, rs, n, desc)
            W = mx.DeviceBuffer(max(ws, 4))
            mx.launch_reduce(op, mx.FLOAT32, rs, n, desc, O.ptr, X.ptr, W.ptr, ws)
            mx.sync()
            if key == "sum":
                got = O.download(np.float32)
                assert np.all(np.abs(got - G[f"red_sum{axis}"]) <= 1e-4 * G[f"red_abs{axis}"])
            else:
                dt = np.int32 if key.startswith("arg") else np.float32
                assert np.array_equal(O.download(dt), G[f"red_{key}{axis}"]), (key, axis)

    ma, bt = G["mm_a"], np.ascontiguousarray(G["mm_b"].T)
    MA, MB = mx.DeviceBuffer.from_numpy(ma), mx.DeviceBuffer.from_numpy(bt)
    MC = mx.DeviceBuffer(2 * 9 * 11 * 4)
    mx.launch_batched_matmul(mx.FLOAT32, ([2, 9, 11], [9 * 13, 13, 1], [0, 13, 1], [9 * 11, 11, 1]), 13,
                             MC.ptr, MA.ptr, MB.ptr)
    mx.sync()
    assert normwise_rel(MC.download(np.float32), G["mm_c"]) <= 1e-4

    ci, ck = G["conv_in"], G["conv_k"]
    geom = dict(in_shape=[2, 6, 5, 3], k_shape=[4, 3, 3, 3], out_shape=[2, 6, 5, 4],
                in_strides=contiguous_strides([2, 6, 5, 3]), k_strides=contiguous_strides([4, 3, 3, 3]),
                out_strides=contiguous_strides([2, 6, 5, 4]), pad=[1, 1], stride=[1, 1])
    CI, CK = mx.DeviceBuffer.from_numpy(ci), mx.DeviceBuffer.from_numpy(ck)
    CO = mx.DeviceBuffer(2 * 6 * 5 * 4 * 4)
    wsb = mx.conv_workspace_bytes(mx.FLOAT32, geom)
    WS = mx.DeviceBuffer(max(wsb, 256))
    mx.launch_conv_nd(mx.FLOAT32, geom, CO.ptr, CI.ptr, CK.ptr, WS.ptr, wsb)
    mx.sync()
    assert normwise_rel(CO.download(np.float32), G["conv_out"]) <= 1e-4

    S = mx.DeviceBuffer.from_numpy(G["cast_src"])
    D = mx.DeviceBuffer(40 * 4)
    mx.launch_copy_strided(mx.INT32, mx.FLOAT32, ([40], [1], [1]), D.ptr, S.ptr)
    mx.sync()
    assert np.array_equal(D.download(np.int32, 40), G["cast_i32"])
    mx.launch_copy_strided(mx.FLOAT16, mx.FLOAT32, ([40], [1], [1]), D.ptr, S.ptr)
    mx.sync()
    assert np.array_equal(D.download(np.uint16, 40), G["cast_f16"])
