"""GPU parity at the workloads' full sizes, checked on sampled outputs.

The oracle's loops at these sizes (7.4 G multiply-adds for the 3x3 convolution, 137 G for the
batched product) would take minutes, so each test runs the full-size launch once and recomputes a
random sample of 4096 of its outputs as the oracle defines them, in float64 from the same stored
inputs: conv_cpu's taps (sample = o * stride - pad + i, Matrix.mm:5705-5736, 12397-12500) and
batched_dot_cpu's K loop (Matrix.mm:7157-7191).  A mistake in the tiling, the tap order, the
padding, the batch walk or the edge tiles shows as sampled outputs far off; the sample covers
every tile with high probability (784 conv tiles, 4096 samples).

Bound per sampled output: |got - ref| <= rel * |ref| + eps * sum_k |a_k b_k|, with rel the output
dtype's rounding (0 for fp32, 2^-10 for float16) and eps 2e-5 for the fp32 accumulation.
"""
import numpy as np
import pytest

from helpers import contiguous_strides

pytestmark = pytest.mark.gpu

SAMPLES = 4096
EPS = 2e-5
REL = {"FLOAT32": 0.0, "FLOAT16": 2.0 ** -10}


def stored(code, x, mx):
    return x.astype(np.float16) if code == mx.FLOAT16 else x.astype(np.float32)


def check_samples(got, ref, mag, rel, what):
    bound = rel * np.abs(ref) + EPS * mag
    bad = np.abs(got.astype(np.float64) - ref) > bound
    assert not bad.any(), (what, int(bad.sum()), float(np.max(np.abs(got - ref) - bound)))


@pytest.mark.parametrize("dt", ["FLOAT32", "FLOAT16"])
@pytest.mark.parametrize("case", [
    # (N, C, H, W, O, k, pad, stride): the NCHW tensors fed as NHWC / OHWI views
    (32, 64, 56, 56, 128, 3, 1, 1),       # 3x3, pad 1
    (32, 256, 28, 28, 512, 1, 0, 2),      # 1x1, stride 2
])
def test_conv2d_full_size_sampled(mx, dt, case):
    code = getattr(mx, dt)
    n, c, h, w, o, k, pad, stride = case
    rng = np.random.default_rng(c * 7 + k)
    x = stored(code, rng.standard_normal([n, c, h, w]).astype(np.float32), mx)
    wt = stored(code, (rng.standard_normal([o, c, k, k]) * np.sqrt(2.0 / (c * k * k))).astype(np.float32), mx)
    oh = (h + 2 * pad - k) // stride + 1
    ow = (w + 2 * pad - k) // stride + 1
    xs, ws = contiguous_strides([n, c, h, w]), contiguous_strides([o, c, k, k])
    in_shape, in_st = [n, h, w, c], [xs[0], xs[2], xs[3], xs[1]]
    k_shape, k_st = [o, k, k, c], [ws[0], ws[2], ws[3], ws[1]]
    out_shape = [n, oh, ow, o]
    total = n * oh * ow * o
    geom = dict(in_shape=in_shape, k_shape=k_shape, out_shape=out_shape, in_strides=in_st, k_strides=k_st,
                out_strides=contiguous_strides(out_shape), pad=[pad, pad], stride=[stride, stride], dil=[1, 1],
                dil_lhs=[1, 1], groups=1, flip=0)
    X = mx.DeviceBuffer.from_numpy(x.reshape(-1))
    W = mx.DeviceBuffer.from_numpy(wt.reshape(-1))
    Y = mx.DeviceBuffer(total * x.itemsize)
    Y.fill_bytes(0xFF)
    wsb = mx.conv_workspace_bytes(code, geom)
    WS = mx.DeviceBuffer(max(wsb, 256))
    mx.launch_conv_nd(code, geom, Y.ptr, X.ptr, W.ptr, WS.ptr, wsb)
    mx.sync()
    y = Y.download(x.dtype, total).reshape(out_shape)
    assert np.isfinite(y.astype(np.float32)).all()
    # sampled outputs, recomputed from the taps
    sn, sh, sw, so = (rng.integers(0, e, SAMPLES) for e in (n, oh, ow, o))
    xf, wf = x.astype(np.float64), wt.astype(np.float64)
    ref = np.zeros(SAMPLES)
    mag = np.zeros(SAMPLES)
    for i in range(k):
        for j in range(k):
            ih, iw = sh * stride - pad + i, sw * stride - pad + j
            ok = (ih >= 0) & (ih < h) & (iw >= 0) & (iw < w)
            xv = xf[sn[:, None], np.arange(c)[None, :], np.clip(ih, 0, h - 1)[:, None], np.clip(iw, 0, w - 1)[:, None]]
            terms = xv * wf[so, :, i, j] * ok[:, None]
            ref += terms.sum(1)
            mag += np.abs(terms).sum(1)
    check_samples(y[sn, sh, sw, so], ref, mag, REL[dt], (dt, case))


@pytest.mark.parametrize("dt", ["FLOAT32", "FLOAT16"])
def test_batched_matmul_full_size_sampled(mx, dt):
    """A[16,2048,2048] x B[2048,2048] (B broadcast over the batch, handed over as packed B^T)."""
    code = getattr(mx, dt)
    rng = np.random.default_rng(5)
    B_, M, K, N = 16, 2048, 2048, 2048
    a = stored(code, (rng.standard_normal([B_, M, K]) / np.sqrt(K)).astype(np.float32), mx)
    bt = stored(code, rng.standard_normal([N, K]).astype(np.float32), mx)
    desc = ([B_, M, N], [M * K, K, 1], [0, K, 1], [M * N, N, 1])
    A = mx.DeviceBuffer.from_numpy(a.reshape(-1))
    Bt = mx.DeviceBuffer.from_numpy(bt.reshape(-1))
    C = mx.DeviceBuffer(B_ * M * N * a.itemsize)
    C.fill_bytes(0xFF)
    mx.launch_batched_matmul(code, desc, K, C.ptr, A.ptr, Bt.ptr)
    mx.sync()
    c = C.download(a.dtype, B_ * M * N).reshape(B_, M, N)
    sb, sm, sn = (rng.integers(0, e, SAMPLES) for e in (B_, M, N))
    terms = a[sb, sm, :].astype(np.float64) * bt[sn, :].astype(np.float64)
    check_samples(c[sb, sm, sn], terms.sum(1), np.abs(terms).sum(1), REL[dt], dt)
    # whole rows and columns at the edges of the tile grid
    for (b, m) in [(0, 0), (15, 2047), (7, 1024)]:
        t = a[b, m, :].astype(np.float64)[None, :] * bt.astype(np.float64)
        check_samples(c[b, m, :], t.sum(1), np.abs(t).sum(1), REL[dt], (dt, "row", b, m))
