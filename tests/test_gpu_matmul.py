"""GPU parity: batched MatMul vs the oracle.

fp32: normwise relative error <= 1e-4 against the oracle (the reference's sequential loop);
fp16 / bf16 with fp32 accumulation: <= 1e-2 normwise against the oracle's fp32-accumulator mode
(same loop, float accumulator, one rounding) -- the literal reference loop accumulates in half,
whose own error at K = 2048 is about that large, so it is reported, not gated;
integer dtypes: exact (wrap-around).  Descriptors come from the product's broadcast +
collapse_dims_matmul helpers, as dot() builds them.
"""
import math

import numpy as np
import pytest

from helpers import bits, contiguous_strides, normwise_rel

pytestmark = pytest.mark.gpu


def matmul_desc(mx, a_shape, a_strides, bt_shape, bt_strides):
    out, out_st, b1s, b1st, b2s, b2st = mx.broadcast_shapes(a_shape, a_strides, bt_shape, bt_strides, matmul=True)
    if len(out) == 2:
        desc = [out, [b1st[0], b1st[1]], [b2st[0], b2st[1]], out_st]
    else:
        desc = mx.collapse_dims_matmul(out, b1st, b2st, out_st)
    return out, desc


def run_mm(mx, orc, code, a, bt, a_shape=None, a_strides=None, bt_shape=None, bt_strides=None, acc=None,
           oracle=True, workspace=True):
    """One product through mx_launch_batched_matmul_ws with the workspace its query asks for
    (workspace=False: the reference-signature entry point, which never splits K)."""
    a_shape = list(a_shape or a.shape)
    bt_shape = list(bt_shape or bt.shape)
    a_strides = a_strides or contiguous_strides(a_shape)
    bt_strides = bt_strides or contiguous_strides(bt_shape)
    out, desc = matmul_desc(mx, a_shape, a_strides, bt_shape, bt_strides)
    K = a_shape[-1]
    total = int(np.prod(out))
    A = mx.DeviceBuffer.from_numpy(a.reshape(-1))
    B = mx.DeviceBuffer.from_numpy(bt.reshape(-1))
    C = mx.DeviceBuffer(total * a.dtype.itemsize)
    wsb = mx.matmul_workspace_bytes(code, desc, K) if workspace else 0
    W = mx.DeviceBuffer(wsb) if wsb else None
    mx.launch_batched_matmul(code, desc, K, C.ptr, A.ptr, B.ptr, workspace=W.ptr if W else 0, workspace_bytes=wsb)
    mx.sync()
    got = C.download(a.dtype, total)
    if not oracle:          # the oracle reads K unit-stride (packed operands)
        return got, None, out
    ref = orc.batched_matmul(code, desc, K, a.reshape(-1), bt.reshape(-1), total,
                             acc=orc.ACC_F32 if acc is None else acc)
    return got, ref, out


def as_f32(code, arr, mx):
    if code == mx.BFLOAT16:
        return (arr.astype(np.uint32) << 16).view(np.float32)
    return arr.astype(np.float32)


def gen(rng, code, shape, scale, mx):
    x = (rng.standard_normal(shape) * scale).astype(np.float32)
    if code == mx.FLOAT16:
        return x.astype(np.float16)
    if code == mx.BFLOAT16:
        from oracle.oracle import f32_to_bf16_bits
        return f32_to_bf16_bits(x)
    return x


TOL = {"FLOAT32": 1e-4, "FLOAT16": 1e-2, "BFLOAT16": 1e-2}


@pytest.mark.parametrize("dt", ["FLOAT32", "FLOAT16", "BFLOAT16"])
@pytest.mark.parametrize("case", [
    ([2, 300, 200], [2, 150, 200]),      # ragged M, N, K (tile edges, K tail)
    ([3, 64, 64], [64, 64]),             # Bt broadcast over the batch (folds into M)
    ([513, 257], [129, 257]),            # rank 2, odd sizes
    ([2, 2, 40, 72], [2, 1, 24, 72]),    # two batch axes, one broadcast
    ([1, 256, 512], [256, 512]),         # exact tiles
])
def test_float_matmul_shapes(mx, orc, dt, case):
    code = getattr(mx, dt)
    rng = np.random.default_rng(10)
    a_shape, bt_shape = case
    K = a_shape[-1]
    a = gen(rng, code, a_shape, 1.0 / math.sqrt(K), mx)
    bt = gen(rng, code, bt_shape, 1.0, mx)
    got, ref, _ = run_mm(mx, orc, code, a, bt)
    assert normwise_rel(as_f32(code, got, mx), as_f32(code, ref, mx)) <= TOL[dt]


@pytest.mark.parametrize("dt", ["FLOAT32", "FLOAT16", "BFLOAT16"])
@pytest.mark.parametrize("K", [200, 201])
def test_large_tiles_ragged(mx, orc, dt, K):
    """256 x 256 tiles (17 x 16 of them) with ragged M and N edges: K = 200 leaves a K tail after
    the DMA'd pairs, K = 201 makes 16-bit rows misaligned so every step goes through the guarded
    element loads (for 16-bit types with eight waves per block).  Checked in fp64 with numpy."""
    code = getattr(mx, dt)
    rng = np.random.default_rng(21)
    M, N = 4100, 4000
    a = gen(rng, code, [M, K], 1.0 / math.sqrt(K), mx)
    bt = gen(rng, code, [N, K], 1.0, mx)
    got, _, _ = run_mm(mx, orc, code, a, bt, oracle=False)
    ref64 = as_f32(code, a, mx).astype(np.float64) @ as_f32(code, bt, mx).astype(np.float64).T
    assert normwise_rel(as_f32(code, got, mx), ref64.reshape(-1)) <= NN_TOL64[dt]


@pytest.mark.parametrize("dt", ["FLOAT32", "FLOAT16"])
def test_main_matmul_shape_reduced_batch(mx, orc, dt):
    """A[2,2048,2048] x B[2048,2048] (B broadcast): the batched-matmul workload's shape at batch 2."""
    code = getattr(mx, dt)
    rng = np.random.default_rng(0)
    a = gen(rng, code, [2, 2048, 2048], 1.0 / math.sqrt(2048), mx)
    bt = gen(rng, code, [2048, 2048], 1.0 / math.sqrt(2048), mx)
    got, ref, _ = run_mm(mx, orc, code, a, bt)
    err = normwise_rel(as_f32(code, got, mx), as_f32(code, ref, mx))
    assert err <= TOL[dt], err


def test_skinny_matmul(mx, orc):
    """A[8,1,4096] x B[4096,4096]: the skinny case (memory bound)."""
    rng = np.random.default_rng(1)
    for code in (mx.FLOAT32, mx.FLOAT16):
        a = gen(rng, code, [8, 1, 4096], 1.0 / 64, mx)
        bt = gen(rng, code, [4096, 4096], 1.0 / 64, mx)
        got, ref, out = run_mm(mx, orc, code, a, bt)
        assert out == [8, 1, 4096]
        tol = 1e-4 if code == mx.FLOAT32 else 1e-2
        assert normwise_rel(as_f32(code, got, mx), as_f32(code, ref, mx)) <= tol


@pytest.mark.parametrize("dt", ["FLOAT32", "FLOAT16", "BFLOAT16"])
@pytest.mark.parametrize("case", [
    ([100, 3000], [70, 3000]),           # one tile, long ragged K: many K splits, short last split
    ([512, 4096], [10, 4096]),           # the MLP's 10-wide output layer
    ([4, 3, 2000], [2000, 2000]),        # batch folded into M, split K
    ([2, 64, 1000], [2, 96, 1000]),      # per-batch Bt, split K with two batches
])
def test_split_k(mx, orc, dt, case):
    """Few output tiles and a long K: the K range is split over blocks and summed in order."""
    code = getattr(mx, dt)
    rng = np.random.default_rng(12)
    a_shape, bt_shape = case
    K = a_shape[-1]
    a = gen(rng, code, a_shape, 1.0 / math.sqrt(K), mx)
    bt = gen(rng, code, bt_shape, 1.0, mx)
    got, ref, _ = run_mm(mx, orc, code, a, bt)
    assert normwise_rel(as_f32(code, got, mx), as_f32(code, ref, mx)) <= TOL[dt]
    got2, _, _ = run_mm(mx, orc, code, a, bt)          # deterministic: the same bits again
    assert np.array_equal(got, got2)


@pytest.mark.parametrize("dt", ["FLOAT32", "FLOAT16"])
def test_split_k_workspace_rules(mx, orc, dt):
    """A product that splits K asks for a workspace; without one (the reference-signature entry
    point, or a workspace one byte short) it runs unsplit, within the same tolerance, and no
    call allocates device memory."""
    code = getattr(mx, dt)
    rng = np.random.default_rng(14)
    a_shape, bt_shape = [512, 4096], [10, 4096]
    a = gen(rng, code, a_shape, 1.0 / 64, mx)
    bt = gen(rng, code, bt_shape, 1.0, mx)
    out, desc = matmul_desc(mx, a_shape, contiguous_strides(a_shape), bt_shape, contiguous_strides(bt_shape))
    wsb = mx.matmul_workspace_bytes(code, desc, 4096)
    assert wsb > 0 and wsb % (512 * 10 * 4) == 0
    before = mx.alloc_stats()
    split, ref, _ = run_mm(mx, orc, code, a, bt)
    plain, _, _ = run_mm(mx, orc, code, a, bt, workspace=False)
    A = mx.DeviceBuffer.from_numpy(a.reshape(-1))
    B = mx.DeviceBuffer.from_numpy(bt.reshape(-1))
    C = mx.DeviceBuffer(512 * 10 * a.dtype.itemsize)
    W = mx.DeviceBuffer(wsb)
    mx.launch_batched_matmul(code, desc, 4096, C.ptr, A.ptr, B.ptr, workspace=W.ptr, workspace_bytes=wsb - 1)
    mx.sync()
    short = C.download(a.dtype, 512 * 10)
    assert np.array_equal(short, plain)                  # one byte short: the unsplit product
    for got in (split, plain):
        assert normwise_rel(as_f32(code, got, mx), as_f32(code, ref, mx)) <= TOL[dt]
    # the only allocations were this test's own buffers: A, B, C and the workspace in the first
    # run_mm, A, B and C in the second, four here
    after = mx.alloc_stats()
    assert after[0] - before[0] == 4 + 3 + 4


@pytest.mark.parametrize("case", [([2048, 2048], [2048, 2048]), ([16, 2048, 2048], [2048, 2048]),
                                  ([8, 1, 4096], [4096, 4096])])
def test_no_workspace_when_tiles_fill_the_chip(mx, case):
    """Products with enough output tiles, and the skinny kernel's shapes, never split."""
    a_shape, bt_shape = case
    out, desc = matmul_desc(mx, a_shape, contiguous_strides(a_shape), bt_shape, contiguous_strides(bt_shape))
    for code in (mx.FLOAT32, mx.FLOAT16, mx.BFLOAT16, mx.INT32):
        assert mx.matmul_workspace_bytes(code, desc, a_shape[-1]) == 0


def test_split_k_strided(mx, orc):
    """A transposed A (scalar-load path) with a split K range."""
    rng = np.random.default_rng(13)
    base = rng.standard_normal([2500, 40]).astype(np.float32)   # A = base.T : [40, 2500], strides [1, 40]
    bt = rng.standard_normal([24, 2500]).astype(np.float32)
    got, _, _ = run_mm(mx, orc, mx.FLOAT32, base, bt, a_shape=[40, 2500], a_strides=[1, 40])
    ref64 = base.T.astype(np.float64) @ bt.T.astype(np.float64)
    assert normwise_rel(got, ref64) <= 1e-5


def test_identity_and_one_hot_exact(mx, orc):
    rng = np.random.default_rng(2)
    a = rng.standard_normal([3, 96, 80]).astype(np.float32)
    eye = np.eye(80, dtype=np.float32)           # Bt = I  ->  C = A exactly
    got, _, _ = run_mm(mx, orc, mx.FLOAT32, a, eye)
    assert np.array_equal(got.reshape(3, 96, 80), a)
    perm = np.eye(80, dtype=np.float32)[rng.permutation(80)]
    got, _, _ = run_mm(mx, orc, mx.FLOAT32, a, perm)
    assert np.array_equal(got.reshape(3, 96, 80), a @ perm.T)


def test_strided_operands(mx, orc):
    """Non-unit K stride (a transposed view) takes the scalar-load path."""
    rng = np.random.default_rng(3)
    base = rng.standard_normal([70, 50]).astype(np.float32)     # A = base.T : [50, 70], strides [1, 50]
    bt = rng.standard_normal([30, 70]).astype(np.float32)
    got, ref, _ = run_mm(mx, orc, mx.FLOAT32, base, bt, a_shape=[50, 70], a_strides=[1, 50])
    ref64 = base.T.astype(np.float64) @ bt.T.astype(np.float64)
    assert normwise_rel(got, ref64) <= 1e-5
    del ref


@pytest.mark.parametrize("dt", ["INT32", "INT8", "INT64", "UINT8", "UINT32", "INT16", "UINT16", "UINT64", "BOOL"])
def test_integer_matmul_exact(mx, orc, dt):
    code = getattr(mx, dt)
    npt = mx.NP_DTYPE[code]
    rng = np.random.default_rng(4)
    if code == mx.BOOL:
        a = rng.integers(0, 2, [2, 17, 9]).astype(np.bool_)
        bt = rng.integers(0, 2, [2, 5, 9]).astype(np.bool_)
    else:
        info = np.iinfo(npt)
        a = rng.integers(info.min, info.max, [2, 17, 9], dtype=npt, endpoint=True)
        bt = rng.integers(info.min, info.max, [2, 5, 9], dtype=npt, endpoint=True)
    got, ref, _ = run_mm(mx, orc, code, a, bt)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("dt", ["FLOAT32", "FLOAT16", "BFLOAT16"])
@pytest.mark.parametrize("case", [
    ([8, 1, 4096], [4096, 4096]),        # the skinny workload (batch folds into M = 8)
    ([16, 3000], [2050, 3000]),          # M = 16, ragged N (scalar stores), K not a step multiple
    ([1, 1024], [2048, 1024]),           # one row
    ([3, 5, 520], [3, 2048, 520]),       # per-batch Bt: blockIdx.y walks the batch
    ([2, 2, 7, 64], [2, 1, 1024, 64]),   # two batch axes, one broadcast; K shorter than the waves' split
    ([4, 40], [4096, 40]),               # K = 40: most waves idle, K tail inside a step
])
def test_skinny_path(mx, orc, dt, case):
    """At most 16 rows of A after folding: the 16 x 16 MFMA streaming kernel."""
    code = getattr(mx, dt)
    rng = np.random.default_rng(14)
    a_shape, bt_shape = case
    K = a_shape[-1]
    a = gen(rng, code, a_shape, 1.0 / math.sqrt(K), mx)
    bt = gen(rng, code, bt_shape, 1.0, mx)
    got, ref, _ = run_mm(mx, orc, code, a, bt)
    assert normwise_rel(as_f32(code, got, mx), as_f32(code, ref, mx)) <= TOL[dt]
    if code == mx.FLOAT32:
        ref64 = np.matmul(a.astype(np.float64), np.swapaxes(bt.astype(np.float64), -1, -2))
        assert normwise_rel(got, ref64.reshape(-1)) <= 1e-5


@pytest.mark.parametrize("M", [16, 8, 3])
def test_skinny_one_hot_exact(mx, orc, M):
    """One-hot A rows pick Bt columns exactly: C[m, n] = Bt[n, k_m], for 16, 8 and 3 rows of A."""
    rng = np.random.default_rng(15 + M)
    K, N = 512, 4096
    ks = rng.integers(0, K, M)
    a = np.zeros([M, K], np.float32)
    a[np.arange(M), ks] = 1.0
    bt = rng.standard_normal([N, K]).astype(np.float32)
    got, _, _ = run_mm(mx, orc, mx.FLOAT32, a, bt)
    assert np.array_equal(got.reshape(M, N), bt[:, ks].T)


NN_TOL64 = {"FLOAT32": 1e-5, "FLOAT16": 2e-3, "BFLOAT16": 1e-2}   # vs fp64 of the same inputs


@pytest.mark.parametrize("dt", ["FLOAT32", "FLOAT16", "BFLOAT16"])
@pytest.mark.parametrize("case", [
    ([8, 1, 4096], [4096, 4096]),        # the skinny workload with B as given ([K, N]): split K
    ([16, 3000], [3000, 2048]),          # M = 16, K not a chunk multiple
    ([1, 1024], [1024, 2056]),           # one row, N not a multiple of the column group
    ([3, 5, 520], [3, 520, 2048]),       # per-batch B: blockIdx.y walks the batch
    ([2, 2, 7, 64], [2, 1, 64, 1024]),   # two batch axes, one broadcast; K shorter than a chunk
    ([4, 40], [40, 4096]),               # K = 40: most waves idle, K tail inside a step
    ([8, 65536], [65536, 64]),           # one column group: K split many ways
    ([2, 8], [8, 16384]),                # no split (enough column groups), K = one fragment
])
def test_skinny_n_major_b(mx, orc, dt, case):
    """At most 16 rows of A with B handed over N-major: the streaming kernel reads whole 128-byte
    lines of B's K rows, split over K when the column groups are few; checked against the oracle on
    the packed Bt the reference's dot() builds and in fp64, with and without the split workspace,
    and run to run bit for bit."""
    code = getattr(mx, dt)
    rng = np.random.default_rng(19)
    a_shape, b_shape = case
    K, N = b_shape[-2], b_shape[-1]
    a = gen(rng, code, a_shape, 1.0 / math.sqrt(K), mx)
    b = gen(rng, code, b_shape, 1.0, mx)
    bst = contiguous_strides(b_shape)
    view = dict(bt_shape=b_shape[:-2] + [N, K], bt_strides=bst[:-2] + [1, N], oracle=False)
    got, _, out = run_mm(mx, orc, code, a, b, **view)
    bt = np.ascontiguousarray(np.swapaxes(b, -1, -2))
    _, desc = matmul_desc(mx, list(a_shape), contiguous_strides(a_shape), list(bt.shape), contiguous_strides(bt.shape))
    ref = orc.batched_matmul(code, desc, K, a.reshape(-1), bt.reshape(-1), int(np.prod(out)), acc=orc.ACC_F32)
    ref64 = np.matmul(as_f32(code, a, mx).astype(np.float64), as_f32(code, b, mx).astype(np.float64)).reshape(-1)
    got1, _, _ = run_mm(mx, orc, code, a, b, workspace=False, **view)
    for g in (got, got1):
        assert normwise_rel(as_f32(code, g, mx), as_f32(code, ref, mx)) <= TOL[dt]
        assert normwise_rel(as_f32(code, g, mx), ref64) <= NN_TOL64[dt]
    got2, _, _ = run_mm(mx, orc, code, a, b, **view)
    assert np.array_equal(got, got2)


@pytest.mark.parametrize("dt", ["FLOAT32", "FLOAT16", "BFLOAT16"])
@pytest.mark.parametrize("M", [16, 8, 3])
def test_skinny_n_major_b_one_hot_exact(mx, orc, dt, M):
    """One-hot A rows pick B rows exactly through the N-major streaming kernel: C[m, :] = B[k_m, :]
    (its staged K rows, column placement and transposing reads)."""
    code = getattr(mx, dt)
    rng = np.random.default_rng(20 + M)
    K, N = 1000, 4096
    ks = rng.integers(0, K, M)
    b = gen(rng, code, [K, N], 1.0, mx)
    a = np.zeros([M, K], b.dtype)
    a[np.arange(M), ks] = np.array([1.0], np.float32).astype(np.float16) if code == mx.FLOAT16 else (
        np.float32(1.0) if code == mx.FLOAT32 else np.uint16(0x3F80))
    got, _, _ = run_mm(mx, orc, code, a, b, bt_shape=[N, K], bt_strides=[1, N], oracle=False)
    assert np.array_equal(got.reshape(M, N), b[ks])


@pytest.mark.parametrize("dt", ["FLOAT32", "FLOAT16", "BFLOAT16"])
@pytest.mark.parametrize("case", [
    ([2, 300, 200], [2, 200, 152]),      # ragged M, K tail, N a multiple of 8 but not of the tile
    ([512, 1024], [1024, 4096]),         # the MLP's first layer (split K)
    ([3, 130, 96], [3, 96, 264]),        # per-batch B
    ([3, 130, 96], [3, 96, 260]),        # N a multiple of 4, not 8: 16-bit takes the strided path
    ([4, 64, 128], [128, 64]),           # B shared by the batch (folds into M)
    ([100, 3000], [3000, 72]),           # long ragged K: split K, short last split
    ([64, 40], [40, 10]),                # N not a multiple of 4: the strided fallback
])
def test_n_major_b(mx, orc, dt, case):
    """B handed over as [..., K, N] (Bt is its transposed view: N stride 1, K stride N): fp32 reads
    it through 16-byte rows of 4 columns, 16-bit types through transposing LDS reads; checked
    against the oracle on the packed Bt the reference's dot() builds, and in fp64."""
    code = getattr(mx, dt)
    rng = np.random.default_rng(16)
    a_shape, b_shape = case
    K, N = b_shape[-2], b_shape[-1]
    a = gen(rng, code, a_shape, 1.0 / math.sqrt(K), mx)
    b = gen(rng, code, b_shape, 1.0, mx)
    bst = contiguous_strides(b_shape)
    bt_shape = b_shape[:-2] + [N, K]
    bt_strides = bst[:-2] + [1, N]
    got, _, out = run_mm(mx, orc, code, a, b, bt_shape=bt_shape, bt_strides=bt_strides, oracle=False)
    # the oracle reads K unit-stride: it gets the packed Bt the reference's dot() would build
    bt = np.ascontiguousarray(np.swapaxes(b, -1, -2))
    _, desc = matmul_desc(mx, list(a_shape), contiguous_strides(a_shape), list(bt.shape), contiguous_strides(bt.shape))
    ref = orc.batched_matmul(code, desc, K, a.reshape(-1), bt.reshape(-1), int(np.prod(out)), acc=orc.ACC_F32)
    assert normwise_rel(as_f32(code, got, mx), as_f32(code, ref, mx)) <= TOL[dt]
    ref64 = np.matmul(as_f32(code, a, mx).astype(np.float64), as_f32(code, b, mx).astype(np.float64))
    assert normwise_rel(as_f32(code, got, mx), ref64.reshape(-1)) <= NN_TOL64[dt]
    got2, _, _ = run_mm(mx, orc, code, a, b, bt_shape=bt_shape, bt_strides=bt_strides, oracle=False)
    assert np.array_equal(got, got2)


@pytest.mark.parametrize("dt", ["FLOAT32", "FLOAT16", "BFLOAT16"])
@pytest.mark.parametrize("case", [
    ([4096, 64], [64, 8192]),            # 256 x 256 tiles
    ([131072, 64], [64, 128]),           # 256 x 128 tiles
])
def test_n_major_b_large_tiles(mx, dt, case):
    """The N-major B slot in the two 256-row tile shapes (checked in fp64 with numpy)."""
    code = getattr(mx, dt)
    rng = np.random.default_rng(17)
    a_shape, b_shape = case
    K, N = b_shape
    a = gen(rng, code, a_shape, 1.0 / math.sqrt(K), mx)
    b = gen(rng, code, b_shape, 1.0, mx)
    M = a_shape[0]
    A = mx.DeviceBuffer.from_numpy(a.reshape(-1))
    B = mx.DeviceBuffer.from_numpy(b.reshape(-1))
    C = mx.DeviceBuffer(M * N * a.itemsize)
    out, desc = matmul_desc(mx, [M, K], [K, 1], [N, K], [1, N])
    mx.launch_batched_matmul(code, desc, K, C.ptr, A.ptr, B.ptr)
    mx.sync()
    got = C.download(a.dtype, M * N)
    ref64 = as_f32(code, a, mx).astype(np.float64) @ as_f32(code, b, mx).astype(np.float64)
    assert normwise_rel(as_f32(code, got, mx), ref64.reshape(-1)) <= NN_TOL64[dt]


@pytest.mark.parametrize("dt", ["FLOAT32", "FLOAT16", "BFLOAT16"])
@pytest.mark.parametrize("MKN", [(300, 200, 152), (1024, 256, 512), (256, 64, 256)])
def test_n_major_b_one_hot_exact(mx, orc, dt, MKN):
    """One-hot A rows pick B rows exactly: C[m, :] = B[k_m, :] (the columns and K rows of the N-major
    slot and the epilogue's placement)."""
    code = getattr(mx, dt)
    M, K, N = MKN
    rng = np.random.default_rng(18)
    ks = rng.integers(0, K, M)
    one = gen(rng, code, [1], 0.0, mx)
    a = np.zeros([M, K], one.dtype)
    a[np.arange(M), ks] = np.array([1.0], np.float32).astype(np.float16) if code == mx.FLOAT16 else (
        np.float32(1.0) if code == mx.FLOAT32 else np.uint16(0x3F80))
    b = gen(rng, code, [K, N], 1.0, mx)
    got, _, _ = run_mm(mx, orc, code, a, b, bt_shape=[N, K], bt_strides=[1, N], oracle=False)
    assert np.array_equal(got.reshape(M, N), b[ks])


@pytest.mark.parametrize("dt", ["FLOAT32", "FLOAT16", "BFLOAT16"])
@pytest.mark.parametrize("b_nmajor", [False, True])
@pytest.mark.parametrize("case", [
    ([2, 200, 304], [2, 200, 152]),      # A^T [.., K, M]: ragged M (multiple of 8), K tail, per-batch B
    ([1024, 512], [1024, 4096]),         # g^T . A of the MLP's first layer shape: split K
    ([96, 4096], [96, 4096]),            # 256 x 256 tiles, K a single pair and a half
    ([3000, 64], [3000, 72]),            # long ragged K: split K, short last split
    ([64, 44], [64, 32]),                # M not a multiple of 8: the strided fallback
])
def test_m_major_a(mx, orc, dt, b_nmajor, case):
    """A handed over M-major (a transposed view of A^T stored [..., K, M], the vjp's g^T):
    16-bit types read it through transposing LDS reads, fp32 through its own fragment layout.  The
    16-bit result must equal the same product on the packed A bit for bit (the fragments are the
    same); every result matches the oracle / fp64 within the usual bounds."""
    code = getattr(mx, dt)
    rng = np.random.default_rng(19)
    at_shape, b_shape = case
    K, M, N = at_shape[-2], at_shape[-1], b_shape[-1]
    at = gen(rng, code, at_shape, 1.0 / math.sqrt(K), mx)
    b = gen(rng, code, b_shape, 1.0, mx)
    ast = contiguous_strides(at_shape)
    a_shape = at_shape[:-2] + [M, K]
    a_strides = ast[:-2] + [1, M]
    bst = contiguous_strides(b_shape)
    bt_shape = b_shape[:-2] + [N, K]
    if b_nmajor:
        bt_store, bt_strides = b, bst[:-2] + [1, N]
    else:
        bt_store = np.ascontiguousarray(np.swapaxes(b, -1, -2))
        bt_strides = contiguous_strides(bt_shape)
    got, _, out = run_mm(mx, orc, code, at, bt_store, a_shape=a_shape, a_strides=a_strides, bt_shape=bt_shape,
                         bt_strides=bt_strides, oracle=False)
    a = np.ascontiguousarray(np.swapaxes(at, -1, -2))
    packed, _, _ = run_mm(mx, orc, code, a, bt_store, bt_shape=bt_shape, bt_strides=bt_strides, oracle=False)
    if M % 8 == 0 and code != mx.FLOAT32:   # the transposed slot: the very fragments of the packed A
        assert np.array_equal(bits(got), bits(packed)), "M-major A differs from the packed A"
    bt = np.ascontiguousarray(np.swapaxes(b, -1, -2))
    _, desc = matmul_desc(mx, list(a.shape), contiguous_strides(list(a.shape)), list(bt.shape),
                          contiguous_strides(list(bt.shape)))
    ref = orc.batched_matmul(code, desc, K, a.reshape(-1), bt.reshape(-1), int(np.prod(out)), acc=orc.ACC_F32)
    assert normwise_rel(as_f32(code, got, mx), as_f32(code, ref, mx)) <= TOL[dt]
    ref64 = np.matmul(as_f32(code, a, mx).astype(np.float64), as_f32(code, b, mx).astype(np.float64))
    assert normwise_rel(as_f32(code, got, mx), ref64.reshape(-1)) <= NN_TOL64[dt]


@pytest.mark.parametrize("dt", ["FLOAT32", "FLOAT16", "BFLOAT16"])
@pytest.mark.parametrize("MKN", [(304, 200, 152), (1024, 256, 512), (256, 64, 256), (4096, 64, 4096)])
def test_m_major_a_one_hot_exact(mx, orc, dt, MKN):
    """One-hot rows of an M-major A pick B rows exactly: C[m, :] = B[k_m, :] (the rows and K rows of
    the transposed A slot and the epilogue's placement)."""
    code = getattr(mx, dt)
    M, K, N = MKN
    rng = np.random.default_rng(20)
    ks = rng.integers(0, K, M)
    if code == mx.FLOAT32:
        at = np.zeros([K, M], np.float32)
        at[ks, np.arange(M)] = 1.0
    else:
        one = np.float16(1.0).view(np.uint16) if code == mx.FLOAT16 else np.uint16(0x3F80)
        at = np.zeros([K, M], np.uint16)
        at[ks, np.arange(M)] = one
        if code == mx.FLOAT16:
            at = at.view(np.float16)
    b = gen(rng, code, [K, N], 1.0, mx)
    bt = np.ascontiguousarray(b.T)
    got, _, _ = run_mm(mx, orc, code, at, bt, a_shape=[M, K], a_strides=[1, M], oracle=False)
    assert np.array_equal(bits(got.reshape(M, N)), bits(b[ks]))
