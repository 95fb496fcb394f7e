"""GPU parity: ConvolutionND (channels-last, mx_launch_conv_nd) vs the oracle.

The oracle is the CPU conv loop (conv_cpu, Matrix.mm:12397-12500).  fp32 through the implicit
GEMM: normwise relative error <= 1e-4; fp16 / bf16 (fp32 accumulation): <= 1e-2 normwise
against the oracle's fp32-accumulator mode.  The direct kernel (integers, input dilation,
3-D) runs the reference's loop order with fma, so its fp32 results must equal the oracle's bit
for bit, and integers are exact.  Inputs are fed as the reference's conv2d sees NCHW tensors
(transposed, strided views) as well as native NHWC.
"""
import numpy as np
import pytest

from helpers import bits, contiguous_strides, normwise_rel

pytestmark = pytest.mark.gpu

TOL = {"FLOAT32": 1e-4, "FLOAT16": 1e-2, "BFLOAT16": 1e-2}


def store_of(code, x, mx):
    if code == mx.FLOAT16:
        return x.astype(np.float16)
    if code == mx.BFLOAT16:
        from oracle.oracle import f32_to_bf16_bits
        return f32_to_bf16_bits(x)
    if code in (mx.INT32,):
        return x.astype(np.int32)
    if code in (mx.INT64,):
        return x.astype(np.int64)
    return x.astype(np.float32)


def out_extent(s, k, pad, stride, dil, dil_lhs):
    span = (s - 1) * dil_lhs + 1
    return (span + 2 * pad - dil * (k - 1) - 1) // stride + 1


def run_conv(mx, orc, code, x_store, in_shape, in_strides, w_store, k_shape, k_strides, pad, stride, dil=None,
             dil_lhs=None, groups=1, flip=0, out_layout="nhwc"):
    ns = len(in_shape) - 2
    dil = dil or [1] * ns
    dil_lhs = dil_lhs or [1] * ns
    os_ = [out_extent(in_shape[d + 1], k_shape[d + 1], pad[d], stride[d], dil[d], dil_lhs[d]) for d in range(ns)]
    out_shape = [in_shape[0]] + os_ + [k_shape[0]]
    if out_layout == "nhwc":
        out_strides = contiguous_strides(out_shape)
    else:                                   # channels-major storage [N, O, spatial..] viewed NHWC
        nchw = [out_shape[0], out_shape[-1]] + os_
        cs = contiguous_strides(nchw)
        out_strides = [cs[0]] + cs[2:] + [cs[1]]
    total = int(np.prod(out_shape))
    geom = dict(in_shape=in_shape, k_shape=k_shape, out_shape=out_shape, in_strides=in_strides,
                k_strides=k_strides, out_strides=out_strides, pad=pad, stride=stride, dil=dil, dil_lhs=dil_lhs,
                groups=groups, flip=flip)
    X = mx.DeviceBuffer.from_numpy(np.ascontiguousarray(x_store).reshape(-1))
    W = mx.DeviceBuffer.from_numpy(np.ascontiguousarray(w_store).reshape(-1))
    esz = x_store.dtype.itemsize
    Y = mx.DeviceBuffer(total * esz)
    Y.fill_bytes(0xFF)
    wsb = mx.conv_workspace_bytes(code, geom)
    WS = mx.DeviceBuffer(max(wsb, 256))
    mx.launch_conv_nd(code, geom, Y.ptr, X.ptr, W.ptr, WS.ptr, wsb)
    mx.sync()
    got = Y.download(x_store.dtype, total)
    ref = orc.conv(code, in_shape, k_shape, out_shape, in_strides, k_strides, out_strides, pad, stride, dil, dil_lhs,
                   groups, flip, np.ascontiguousarray(x_store).reshape(-1), np.ascontiguousarray(w_store).reshape(-1),
                   total)
    return got, ref


def as_f32(code, a, mx):
    if code == mx.BFLOAT16:
        return (a.astype(np.uint32) << 16).view(np.float32)
    return a.astype(np.float32)


def nchw_view(n, c, h, w):
    """shape / strides of an NCHW tensor seen as NHWC (transpose(0, 2, 3, 1))."""
    st = contiguous_strides([n, c, h, w])
    return [n, h, w, c], [st[0], st[2], st[3], st[1]]


def oihw_view(o, i, kh, kw):
    st = contiguous_strides([o, i, kh, kw])
    return [o, kh, kw, i], [st[0], st[2], st[3], st[1]]


@pytest.mark.parametrize("dt", ["FLOAT32", "FLOAT16", "BFLOAT16"])
@pytest.mark.parametrize("case", [
    # (N, C, H, W, O, kh, kw, pad, stride, layout)
    (2, 64, 9, 11, 32, 3, 3, 1, 1, "nchw"),        # 3x3 pad 1 on NCHW views (config 4, scaled)
    (2, 64, 9, 7, 48, 3, 3, 1, 2, "nhwc"),         # native NHWC, stride 2
    (2, 128, 12, 12, 64, 1, 1, 0, 2, "nchw"),      # 1x1 stride 2 (config 4's second case, scaled)
    (1, 3, 10, 10, 16, 3, 3, 1, 1, "nhwc"),        # 3 channels: zero-padded K pair
    (3, 64, 6, 6, 160, 3, 3, 1, 1, "nhwc"),        # O > 128: 256-wide N tiles
    (1, 96, 5, 5, 8, 5, 5, 2, 1, "nchw"),          # kernel as large as the image
    (2, 64, 28, 28, 32, 3, 3, 1, 1, "nchw"),       # NCHW pack with 16-byte register transposes
    (2, 20, 8, 8, 16, 3, 3, 1, 1, "nchw"),         # the same with zero channels C..Cgp
])
def test_conv2d_mfma(mx, orc, dt, case):
    code = getattr(mx, dt)
    n, c, h, w, o, kh, kw, pad, stride, layout = case
    rng = np.random.default_rng(n * 100003 + c * 1009 + h * 101 + w * 11 + o + kh)
    if layout == "nchw":
        x = store_of(code, rng.standard_normal([n, c, h, w]).astype(np.float32), mx)
        in_shape, in_st = nchw_view(n, c, h, w)
        wt = store_of(code, (rng.standard_normal([o, c, kh, kw]) * np.sqrt(2.0 / (c * kh * kw))).astype(np.float32), mx)
        k_shape, k_st = oihw_view(o, c, kh, kw)
    else:
        x = store_of(code, rng.standard_normal([n, h, w, c]).astype(np.float32), mx)
        in_shape, in_st = [n, h, w, c], contiguous_strides([n, h, w, c])
        wt = store_of(code, (rng.standard_normal([o, kh, kw, c]) * np.sqrt(2.0 / (c * kh * kw))).astype(np.float32), mx)
        k_shape, k_st = [o, kh, kw, c], contiguous_strides([o, kh, kw, c])
    got, ref = run_conv(mx, orc, code, x, in_shape, in_st, wt, k_shape, k_st, [pad, pad], [stride, stride])
    err = normwise_rel(as_f32(code, got, mx), as_f32(code, ref, mx))
    assert err <= TOL[dt], (dt, case, err)


@pytest.mark.parametrize("dt", ["FLOAT32", "FLOAT16", "BFLOAT16"])
@pytest.mark.parametrize("case", [
    # (N, C, H, W, O, stride_h, stride_w, layout): 1 x 1 kernels, no padding, stride > 1 -- only
    # the sampled positions are packed, then a stride-1 product over them
    (3, 20, 13, 11, 24, 3, 3, "nchw"),     # odd extents, channels zero-padded to the K pair
    (2, 40, 9, 9, 16, 2, 2, "nhwc"),       # channels-last input with padded channels (40 -> 64 / 64 / 64)
    (2, 48, 10, 12, 40, 2, 1, "nchw"),     # stride 2 along H only
    (1, 16, 7, 16, 8, 1, 4, "nhwc"),       # stride 4 along W only
    (2, 130, 30, 29, 24, 2, 2, "nchw"),    # channel-major pack: 4 x 3 position / channel blocks, ragged
])
def test_conv2d_1x1_strided_sampled_pack(mx, orc, dt, case):
    code = getattr(mx, dt)
    n, c, h, w, o, sh, sw, layout = case
    rng = np.random.default_rng(n * 31 + c + o)
    if layout == "nchw":
        x = store_of(code, rng.standard_normal([n, c, h, w]).astype(np.float32), mx)
        in_shape, in_st = nchw_view(n, c, h, w)
        wt = store_of(code, (rng.standard_normal([o, c, 1, 1]) * np.sqrt(2.0 / c)).astype(np.float32), mx)
        k_shape, k_st = oihw_view(o, c, 1, 1)
    else:
        x = store_of(code, rng.standard_normal([n, h, w, c]).astype(np.float32), mx)
        in_shape, in_st = [n, h, w, c], contiguous_strides([n, h, w, c])
        wt = store_of(code, (rng.standard_normal([o, 1, 1, c]) * np.sqrt(2.0 / c)).astype(np.float32), mx)
        k_shape, k_st = [o, 1, 1, c], contiguous_strides([o, 1, 1, c])
    got, ref = run_conv(mx, orc, code, x, in_shape, in_st, wt, k_shape, k_st, [0, 0], [sh, sw])
    err = normwise_rel(as_f32(code, got, mx), as_f32(code, ref, mx))
    assert err <= TOL[dt], (dt, case, err)
    # the same product as a stride-1 convolution over the sampled positions taken as a strided
    # view: the ordinary pack path and one GEMM of the same M, N and K -- equal bit for bit
    view_shape = [n, (h - 1) // sh + 1, (w - 1) // sw + 1, c]
    view_st = [in_st[0], in_st[1] * sh, in_st[2] * sw, in_st[3]]
    got1, _ = run_conv(mx, orc, code, x, view_shape, view_st, wt, k_shape, k_st, [0, 0], [1, 1])
    assert np.array_equal(bits(got), bits(got1)), (dt, case)


@pytest.mark.parametrize("dt", ["FLOAT32", "FLOAT16"])
def test_conv1d_1x1_strided_sampled_pack(mx, orc, dt):
    code = getattr(mx, dt)
    rng = np.random.default_rng(17)
    n, c, L, o, s = 3, 36, 101, 20, 3
    x = store_of(code, rng.standard_normal([n, c, L]).astype(np.float32), mx)
    st = contiguous_strides([n, c, L])
    wt = store_of(code, (rng.standard_normal([o, 1, c]) * np.sqrt(2.0 / c)).astype(np.float32), mx)
    got, ref = run_conv(mx, orc, code, x, [n, L, c], [st[0], st[2], st[1]], wt, [o, 1, c],
                        contiguous_strides([o, 1, c]), [0], [s])
    err = normwise_rel(as_f32(code, got, mx), as_f32(code, ref, mx))
    assert err <= TOL[dt], (dt, err)


@pytest.mark.parametrize("dt", ["FLOAT32", "FLOAT16"])
def test_conv2d_groups_dilation_flip_strided_output(mx, orc, dt):
    code = getattr(mx, dt)
    rng = np.random.default_rng(7)
    n, h, w, c, o, g = 2, 10, 9, 64, 32, 2
    x = store_of(code, rng.standard_normal([n, h, w, c]).astype(np.float32), mx)
    wt = store_of(code, (rng.standard_normal([o, 3, 3, c // g]) * 0.2).astype(np.float32), mx)
    for kw_args in (dict(groups=2), dict(dil=[2, 2]), dict(flip=1), dict(out_layout="nchw"),
                    dict(groups=2, dil=[2, 1], flip=1, out_layout="nchw")):
        gg = kw_args.get("groups", 1)
        wt_g = wt if gg == 2 else store_of(code, (rng.standard_normal([o, 3, 3, c]) * 0.2).astype(np.float32), mx)
        got, ref = run_conv(mx, orc, code, x, [n, h, w, c], contiguous_strides([n, h, w, c]), wt_g,
                            list(wt_g.shape), contiguous_strides(list(wt_g.shape)), [2, 2], [1, 1], **kw_args)
        err = normwise_rel(as_f32(code, got, mx), as_f32(code, ref, mx))
        assert err <= TOL[dt], (dt, kw_args, err)


@pytest.mark.parametrize("dt", ["FLOAT32", "FLOAT16"])
def test_conv1d_mfma(mx, orc, dt):
    code = getattr(mx, dt)
    rng = np.random.default_rng(3)
    x = store_of(code, rng.standard_normal([3, 50, 64]).astype(np.float32), mx)
    wt = store_of(code, (rng.standard_normal([40, 5, 64]) * 0.1).astype(np.float32), mx)
    got, ref = run_conv(mx, orc, code, x, [3, 50, 64], contiguous_strides([3, 50, 64]), wt, [40, 5, 64],
                        contiguous_strides([40, 5, 64]), [2], [1])
    assert normwise_rel(as_f32(code, got, mx), as_f32(code, ref, mx)) <= TOL[dt]


@pytest.mark.parametrize("dt", ["FLOAT16", "BFLOAT16"])
@pytest.mark.parametrize("case", [
    # (N, H, W, C, O, kh, kw, pad_h, pad_w): more 128 x 128 output tiles than the GPU has CUs, so a
    # block computes several tiles and fetches the next tile's K pairs while it finishes the last
    (8, 50, 50, 64, 160, 1, 1, 0, 0),      # 1 K pair per tile, 314 tiles; O = 160: edge tiles in N
    (5, 64, 64, 128, 144, 1, 1, 0, 0),     # 2 K pairs, 320 tiles
    (9, 64, 64, 64, 64, 1, 3, 0, 1),       # 3 K pairs (one per tap), 288 tiles
    (9, 64, 64, 32, 64, 3, 3, 1, 1),       # 9 K pairs (32 channels, zero-padded to the pair), 288 tiles
])
def test_conv2d_many_tiles(mx, orc, dt, case):
    code = getattr(mx, dt)
    n, h, w, c, o, kh, kw, ph, pw = case
    rng = np.random.default_rng(n * 7919 + c * 31 + o + kw)
    x = store_of(code, rng.standard_normal([n, h, w, c]).astype(np.float32), mx)
    wt = store_of(code, (rng.standard_normal([o, kh, kw, c]) * np.sqrt(2.0 / (c * kh * kw))).astype(np.float32), mx)
    got, ref = run_conv(mx, orc, code, x, [n, h, w, c], contiguous_strides([n, h, w, c]), wt, [o, kh, kw, c],
                        contiguous_strides([o, kh, kw, c]), [ph, pw], [1, 1])
    err = normwise_rel(as_f32(code, got, mx), as_f32(code, ref, mx))
    assert err <= TOL[dt], (dt, case, err)


@pytest.mark.parametrize("dt", ["FLOAT16", "BFLOAT16"])
@pytest.mark.parametrize("case", [
    # (N, H, W, C, O, kh, kw, pad, dil): same convolutions (stride 1, output extents = input
    # extents) over at most 64 channels and 9 kernel positions -- the weight-resident halo kernel.
    # O a multiple of 128 takes its staged whole-row stores; others its per-element edge stores.
    (4, 30, 70, 64, 128, 3, 3, 1, 1),      # 8400 positions: 132 tiles, the last one 16 rows
    (5, 64, 64, 64, 128, 1, 3, 1, 1),      # 320 tiles: blocks walk two tiles through the ring
    (1, 20, 21, 48, 256, 3, 3, 2, 2),      # dilation 2, two full column groups, 48 -> 64 channels
    (1, 6, 150, 64, 128, 3, 3, 1, 1),      # 150-pixel rows: a 368-row halo per tile
    (2, 13, 17, 64, 200, 3, 3, 1, 1),      # a full column group and a 72-channel one
])
def test_conv2d_same_halo(mx, orc, dt, case):
    code = getattr(mx, dt)
    n, h, w, c, o, kh, kw, pad, dil = case
    rng = np.random.default_rng(n * 131 + h * 17 + w + c + o + kw)
    x = store_of(code, rng.standard_normal([n, h, w, c]).astype(np.float32), mx)
    wt = store_of(code, (rng.standard_normal([o, kh, kw, c]) * np.sqrt(2.0 / (c * kh * kw))).astype(np.float32), mx)
    pads = [pad if kh > 1 else 0, pad if kw > 1 else 0]
    got, ref = run_conv(mx, orc, code, x, [n, h, w, c], contiguous_strides([n, h, w, c]), wt, [o, kh, kw, c],
                        contiguous_strides([o, kh, kw, c]), pads, [1, 1], dil=[dil, dil])
    assert got.size == n * h * w * o
    err = normwise_rel(as_f32(code, got, mx), as_f32(code, ref, mx))
    assert err <= TOL[dt], (dt, case, err)


def test_conv1d_same_halo_full_columns(mx, orc):
    code = mx.FLOAT16
    rng = np.random.default_rng(12)
    x = store_of(code, rng.standard_normal([3, 200, 64]).astype(np.float32), mx)
    wt = store_of(code, (rng.standard_normal([128, 5, 64]) * 0.1).astype(np.float32), mx)
    got, ref = run_conv(mx, orc, code, x, [3, 200, 64], contiguous_strides([3, 200, 64]), wt, [128, 5, 64],
                        contiguous_strides([128, 5, 64]), [2], [1])
    assert normwise_rel(as_f32(code, got, mx), as_f32(code, ref, mx)) <= TOL["FLOAT16"]


def test_conv1d_many_tiles(mx, orc):
    code = mx.FLOAT16
    rng = np.random.default_rng(11)
    x = store_of(code, rng.standard_normal([40, 1000, 64]).astype(np.float32), mx)
    wt = store_of(code, (rng.standard_normal([72, 3, 64]) * 0.1).astype(np.float32), mx)
    got, ref = run_conv(mx, orc, code, x, [40, 1000, 64], contiguous_strides([40, 1000, 64]), wt, [72, 3, 64],
                        contiguous_strides([72, 3, 64]), [1], [1])
    assert normwise_rel(as_f32(code, got, mx), as_f32(code, ref, mx)) <= TOL["FLOAT16"]


def test_direct_fp32_is_bit_exact(mx, orc):
    """Input dilation and a 3-D conv take the direct kernel: same loop order as the CPU."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal([2, 7, 6, 5]).astype(np.float32)
    wt = rng.standard_normal([4, 3, 3, 5]).astype(np.float32)
    got, ref = run_conv(mx, orc, mx.FLOAT32, x, [2, 7, 6, 5], contiguous_strides([2, 7, 6, 5]), wt, [4, 3, 3, 5],
                        contiguous_strides([4, 3, 3, 5]), [1, 2], [1, 2], dil_lhs=[2, 3], flip=1)
    assert np.array_equal(bits(got), bits(ref))
    x3 = rng.standard_normal([1, 4, 5, 6, 8]).astype(np.float32)
    w3 = rng.standard_normal([4, 3, 3, 3, 8]).astype(np.float32)
    got, ref = run_conv(mx, orc, mx.FLOAT32, x3, [1, 4, 5, 6, 8], contiguous_strides([1, 4, 5, 6, 8]), w3,
                        [4, 3, 3, 3, 8], contiguous_strides([4, 3, 3, 3, 8]), [1, 1, 1], [1, 2, 1])
    assert np.array_equal(bits(got), bits(ref))


@pytest.mark.parametrize("dt", ["INT32", "INT64"])
def test_integer_conv_exact(mx, orc, dt):
    code = getattr(mx, dt)
    rng = np.random.default_rng(11)
    npdt = np.int32 if dt == "INT32" else np.int64
    x = rng.integers(-50, 50, [2, 6, 5, 7]).astype(npdt)
    wt = rng.integers(-9, 9, [6, 3, 2, 7]).astype(npdt)
    got, ref = run_conv(mx, orc, code, x, [2, 6, 5, 7], contiguous_strides([2, 6, 5, 7]), wt, [6, 3, 2, 7],
                        contiguous_strides([6, 3, 2, 7]), [1, 0], [1, 1])
    assert np.array_equal(got, ref)


def test_workspace_too_small_is_an_error(mx):
    in_shape, in_st = nchw_view(1, 64, 8, 8)
    geom = dict(in_shape=in_shape, k_shape=[8, 3, 3, 64], out_shape=[1, 8, 8, 8], in_strides=in_st,
                k_strides=contiguous_strides([8, 3, 3, 64]), out_strides=contiguous_strides([1, 8, 8, 8]),
                pad=[1, 1], stride=[1, 1])
    need = mx.conv_workspace_bytes(mx.FLOAT32, geom)
    assert need > 0
    X = mx.DeviceBuffer(64 * 64 * 4)
    W = mx.DeviceBuffer(8 * 9 * 64 * 4)
    Y = mx.DeviceBuffer(8 * 64 * 4)
    with pytest.raises(mx.MatrixAMDError) as e:
        mx.launch_conv_nd(mx.FLOAT32, geom, Y.ptr, X.ptr, W.ptr, 0, 0)
    assert e.value.status == mx.ERR_WORKSPACE
