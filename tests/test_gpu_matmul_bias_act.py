"""GPU parity: mx_launch_batched_matmul_bias_act -- a Dot node, a broadcast Add of a bias row and a
Max / Min against a scalar in one call.

C, Z = C + bias and H = max|min(Z, s) must equal mx_launch_batched_matmul followed by two
mx_launch_bcast_binary launches bit for bit (the same product, then the broadcast kernels'
per-element Add and select), on every path of the product: the split-K combine (which writes all
three), the skinny kernel, the unsplit tile kernel with the 16-byte and the one-element epilogue,
per-batch Bt and a batch folded into M.  C itself is checked against the oracle.
"""
import numpy as np
import pytest

from helpers import bits, contiguous_strides, normwise_rel
from test_gpu_matmul import TOL, as_f32, gen, matmul_desc

pytestmark = pytest.mark.gpu

CASES = [
    ([512, 1024], [4096, 1024]),        # the MLP's first layer: split K, combine + epilogue
    ([8, 256], [2048, 256]),            # at most 16 rows of A: skinny kernel, then the epilogue
    ([2048, 256], [2048, 256]),         # 256 tiles, no split: tile kernel, 16-byte epilogue
    ([300, 200], [150, 200]),           # N % 8 != 0, no split: one-element epilogue
    ([2, 300, 200], [2, 152, 200]),     # per-batch Bt
    ([4, 64, 128], [96, 128]),          # Bt shared by the batch: folds into M
]


def np_dtype(mx, code):
    return mx.NP_DTYPE[code]


def scalar_bits(mx, code, v):
    x = np.array([v], np.float32)
    if code == mx.FLOAT16:
        return x.astype(np.float16)
    if code == mx.BFLOAT16:
        from oracle.oracle import f32_to_bf16_bits
        return f32_to_bf16_bits(x)
    return x


def unfused(mx, code, desc, K, out, A, Bt, bias, s, act, total, esz, W, wsb):
    """The three launches the fused call replaces (the product with the same workspace, so it
    splits K exactly as the fused call does)."""
    C = mx.DeviceBuffer(total * esz)
    Z = mx.DeviceBuffer(total * esz)
    H = mx.DeviceBuffer(total * esz)
    mx.launch_batched_matmul(code, desc, K, C.ptr, A.ptr, Bt.ptr, workspace=W.ptr if W else 0, workspace_bytes=wsb)
    N = out[-1]
    bd = mx.broadcast_shapes(list(out), contiguous_strides(out), [N], [1])
    d3 = mx.collapse_dims3(bd[2], bd[3], bd[5], bd[1])
    mx.launch_bcast_binary(mx.OP_ADD, code, d3, Z.ptr, C.ptr, bias.ptr)
    bs = mx.broadcast_shapes(list(out), contiguous_strides(out), [], [])
    ds = mx.collapse_dims3(bs[2], bs[3], bs[5], bs[1])
    mx.launch_bcast_binary(act, code, ds, H.ptr, Z.ptr, s.ptr)
    return C, Z, H


@pytest.mark.parametrize("dt", ["FLOAT32", "FLOAT16", "BFLOAT16"])
@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("act,sval", [("OP_MAX", 0.0), ("OP_MIN", 0.25)])
def test_bias_act_equals_three_launches(mx, orc, dt, case, act, sval):
    code, act_op = getattr(mx, dt), getattr(mx, act)
    rng = np.random.default_rng(len(case[0]) * 100 + case[0][-1])
    a_shape, bt_shape = case
    K = a_shape[-1]
    a = gen(rng, code, a_shape, 1.0 / np.sqrt(K), mx)
    bt = gen(rng, code, bt_shape, 1.0, mx)
    out, desc = matmul_desc(mx, a_shape, contiguous_strides(a_shape), bt_shape, contiguous_strides(bt_shape))
    total = int(np.prod(out))
    N = out[-1]
    bias_h = gen(rng, code, [N], 0.5, mx)
    esz = np.dtype(np_dtype(mx, code)).itemsize
    A = mx.DeviceBuffer.from_numpy(a.reshape(-1))
    Bt = mx.DeviceBuffer.from_numpy(bt.reshape(-1))
    bias = mx.DeviceBuffer.from_numpy(bias_h)
    s = mx.DeviceBuffer.from_numpy(scalar_bits(mx, code, sval))
    C, Z, H = (mx.DeviceBuffer(total * esz) for _ in range(3))
    for B in (C, Z, H):
        B.fill_bytes(0xA5)
    wsb = mx.matmul_workspace_bytes(code, desc, K)
    W = mx.DeviceBuffer(wsb) if wsb else None
    mx.launch_batched_matmul_bias_act(code, desc, K, C.ptr, A.ptr, Bt.ptr, bias.ptr, Z.ptr, act_op, s.ptr, H.ptr,
                                      workspace=W.ptr if W else 0, workspace_bytes=wsb)
    C1, Z1, H1 = unfused(mx, code, desc, K, out, A, Bt, bias, s, act_op, total, esz, W, wsb)
    mx.sync()
    npt = np_dtype(mx, code)
    got = [X.download(npt, total) for X in (C, Z, H)]
    ref = [X.download(npt, total) for X in (C1, Z1, H1)]
    for name, g, r in zip("CZH", got, ref):
        assert np.array_equal(bits(g), bits(r)), (dt, case, act, name)
    # the activation did something: some elements clamped, some passed through
    zf, hf = as_f32(code, got[1], mx), as_f32(code, got[2], mx)
    assert 0 < np.count_nonzero(zf != hf) < total
    # and the product itself is the oracle's
    oref = orc.batched_matmul(code, desc, K, a.reshape(-1), bt.reshape(-1), total, acc=orc.ACC_F32)
    assert normwise_rel(as_f32(code, got[0], mx), as_f32(code, oref, mx)) <= TOL[dt]


def test_bias_act_errors(mx):
    code = mx.FLOAT32
    a_shape, bt_shape = [64, 32], [64, 32]
    out, desc = matmul_desc(mx, a_shape, contiguous_strides(a_shape), bt_shape, contiguous_strides(bt_shape))
    bufs = [mx.DeviceBuffer(64 * 64 * 4) for _ in range(6)]
    p = [b.ptr for b in bufs]
    with pytest.raises(mx.MatrixAMDError) as e:       # integer dtypes have no fused form
        mx.launch_batched_matmul_bias_act(mx.INT32, desc, 32, *p[:3], p[3], p[4], mx.OP_MAX, p[5], p[4])
    assert e.value.status == mx.ERR_UNSUPPORTED
    with pytest.raises(mx.MatrixAMDError):            # only Max / Min
        mx.launch_batched_matmul_bias_act(code, desc, 32, *p[:3], p[3], p[4], mx.OP_ADD, p[5], p[4])
    strided = (desc[0], desc[1], desc[2], [128, 1])   # C rows 128 apart: not contiguous
    with pytest.raises(mx.MatrixAMDError):
        mx.launch_batched_matmul_bias_act(code, strided, 32, *p[:3], p[3], p[4], mx.OP_MAX, p[5], p[4])
    with pytest.raises(mx.MatrixAMDError):            # missing bias
        mx.launch_batched_matmul_bias_act(code, desc, 32, *p[:3], 0, p[4], mx.OP_MAX, p[5], p[4])
