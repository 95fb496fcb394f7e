"""GPU parity: strided copy with dtype cast (mx_launch_copy_strided) vs the oracle.

The oracle restates copyCPUinplaceTypeCasted (matrix.h:1337-1550): static_cast per element,
float -> integer saturating with truncation (arm64 semantics), bool as (x != 0).  Results must
match bit for bit (a NaN may differ only in its payload / sign).
"""
import numpy as np
import pytest

from helpers import bits, contiguous_strides

pytestmark = pytest.mark.gpu

NP = {"FLOAT32": np.float32, "FLOAT16": np.float16, "UINT8": np.uint8, "INT32": np.int32, "INT16": np.int16,
      "UINT32": np.uint32, "UINT16": np.uint16, "BOOL": np.uint8, "INT8": np.int8, "BFLOAT16": np.uint16,
      "INT64": np.int64, "UINT64": np.uint64}
FLOATS = {"FLOAT32", "FLOAT16", "BFLOAT16"}


def values(name, n, rng):
    """Inputs with the edge cases of each type: NaN / inf / huge / negative / fractional."""
    if name in FLOATS:
        v = rng.standard_normal(n).astype(np.float32) * 100
        special = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 3e9, -3e9, 1e20, -1e20, 0.5, -0.5, 255.9,
                            -1.0, 65504.0, 70000.0, 2.0**31, -2.0**31, 2.0**63, 1.5e-5], np.float32)
        v[:len(special)] = special
        if name == "FLOAT16":
            with np.errstate(over="ignore"):
                return v.astype(np.float16)
        if name == "BFLOAT16":
            from oracle.oracle import f32_to_bf16_bits
            return f32_to_bf16_bits(v)
        return v
    info = np.iinfo(NP[name]) if name != "BOOL" else None
    if name == "BOOL":
        return rng.integers(0, 2, n).astype(np.uint8)
    v = rng.integers(info.min, info.max, n, dtype=NP[name], endpoint=True)
    v[:4] = [info.min, info.max, 0, 1]
    return v


def compare(dst_name, got, ref):
    if dst_name in FLOATS:
        if dst_name == "FLOAT32":
            gf, rf = got.astype(np.float32), ref.astype(np.float32)
        elif dst_name == "FLOAT16":
            gf, rf = got.astype(np.float32), ref.astype(np.float32)
        else:
            gf = (got.astype(np.uint32) << 16).view(np.float32)
            rf = (ref.astype(np.uint32) << 16).view(np.float32)
        both_nan = np.isnan(gf) & np.isnan(rf)
        same = bits(got) == bits(ref)
        bad = ~(same | both_nan)
    else:
        bad = bits(got) != bits(ref)
    assert not bad.any(), (dst_name, np.nonzero(bad)[0][:10], got[bad][:5], ref[bad][:5])


@pytest.mark.parametrize("src", list(NP))
@pytest.mark.parametrize("dst", list(NP))
def test_cast_every_pair(mx, orc, src, dst):
    rng = np.random.default_rng(len(src) * 31 + len(dst))
    n = 1000
    x = values(src, n, rng)
    desc = ([n], [1], [1])
    X = mx.DeviceBuffer.from_numpy(x)
    Y = mx.DeviceBuffer(n * np.dtype(NP[dst]).itemsize)
    mx.launch_copy_strided(getattr(mx, dst), getattr(mx, src), desc, Y.ptr, X.ptr)
    mx.sync()
    got = Y.download(NP[dst], n)
    ref = orc.copy_strided(getattr(orc, orc_code(dst)), getattr(orc, orc_code(src)), [n], [1], [1],
                           np.zeros(n, NP[dst]), x)
    compare(dst, got, ref)


def orc_code(name):
    return {"FLOAT32": "F32", "FLOAT16": "F16", "UINT8": "U8", "INT32": "I32", "INT16": "I16", "UINT32": "U32",
            "UINT16": "U16", "BOOL": "BOOL", "INT8": "I8", "BFLOAT16": "BF16", "INT64": "I64",
            "UINT64": "U64"}[name]


@pytest.mark.parametrize("shape,perm", [
    ([64, 48], (1, 0)),                  # 2-D transpose
    ([4, 5, 6, 7], (0, 2, 3, 1)),        # NCHW -> NHWC
    ([3, 128, 40], (0, 1, 2)),           # contiguous rows: 16-byte path
    ([2, 3, 4, 5, 6], (4, 0, 3, 1, 2)),
])
@pytest.mark.parametrize("dt", ["FLOAT32", "FLOAT16", "INT8", "INT64"])
def test_strided_views(mx, orc, shape, perm, dt):
    rng = np.random.default_rng(1)
    x = values(dt, int(np.prod(shape)), rng)
    st = contiguous_strides(shape)
    vshape = [shape[p] for p in perm]
    vst = [st[p] for p in perm]
    dst_st = contiguous_strides(vshape)
    desc = mx.collapse_dims2(vshape, dst_st, vst)
    X = mx.DeviceBuffer.from_numpy(x)
    Y = mx.DeviceBuffer(x.nbytes)
    code = getattr(mx, dt)
    mx.launch_copy_strided(code, code, desc, Y.ptr, X.ptr)
    mx.sync()
    got = Y.download(x.dtype, x.size)
    want = x.reshape(shape).transpose(perm).ravel()
    assert np.array_equal(bits(got), bits(want))


def test_rank0_and_empty(mx, orc):
    x = np.array([3.75], np.float32)
    X = mx.DeviceBuffer.from_numpy(x)
    Y = mx.DeviceBuffer(4)
    mx.launch_copy_strided(mx.INT32, mx.FLOAT32, ([], [], []), Y.ptr, X.ptr)
    mx.sync()
    assert Y.download(np.int32, 1)[0] == 3
    mx.launch_copy_strided(mx.INT32, mx.FLOAT32, ([0], [1], [1]), Y.ptr, X.ptr)   # nothing to do
    mx.sync()


@pytest.mark.parametrize("shape,perm", [
    ([512, 4096], (1, 0)),               # an activation transpose of the MLP step
    ([136, 200], (1, 0)),                # ragged grid in both plane axes
    ([3, 256, 96], (0, 2, 1)),           # batched transpose (batch on blockIdx.z)
    ([2, 40, 3, 64], (0, 3, 1, 2)),      # batch axes on both sides of the plane
    ([10, 4096], (1, 0)),                # unaligned extent: scalar kernel
])
@pytest.mark.parametrize("dt", ["FLOAT32", "FLOAT16", "INT64", "UINT16", "INT32"])
def test_transposes(mx, orc, shape, perm, dt):
    """Same-dtype transposed copies (dot()'s B^T): 16-byte register-block transposes when
    extents and strides are whole 16-byte units, the scalar kernel otherwise."""
    rng = np.random.default_rng(2)
    x = values(dt, int(np.prod(shape)), rng)
    st = contiguous_strides(shape)
    vshape = [shape[p] for p in perm]
    vst = [st[p] for p in perm]
    desc = mx.collapse_dims2(vshape, contiguous_strides(vshape), vst)
    X = mx.DeviceBuffer.from_numpy(x)
    Y = mx.DeviceBuffer(x.nbytes)
    code = getattr(mx, dt)
    mx.launch_copy_strided(code, code, desc, Y.ptr, X.ptr)
    mx.sync()
    got = Y.download(x.dtype, x.size)
    assert np.array_equal(bits(got), bits(x.reshape(shape).transpose(perm).ravel()))


@pytest.mark.parametrize("shape,perm", [
    ([64, 48], (1, 0)),                  # 16-byte register-block transpose
    ([3, 128, 40], (0, 1, 2)),           # contiguous rows: 16-byte path
    ([2, 3, 4, 5, 6], (4, 0, 3, 1, 2)),  # gather
    ([10, 4097], (1, 0)),                # odd extent: gather
])
def test_complex64_views_move_bits(mx, orc, shape, perm):
    """complex64 -> complex64 moves the 8 bytes of every element (NaN payloads and -0 kept)."""
    rng = np.random.default_rng(5)
    n = int(np.prod(shape))
    x = rng.standard_normal(2 * n).astype(np.float32)
    x[:6] = [np.nan, -0.0, np.inf, -np.inf, 1e-45, -3.0]
    x = x.view(np.complex64)
    st = contiguous_strides(shape)
    vshape = [shape[p] for p in perm]
    desc = mx.collapse_dims2(vshape, contiguous_strides(vshape), [st[p] for p in perm])
    X = mx.DeviceBuffer.from_numpy(x)
    Y = mx.DeviceBuffer(x.nbytes)
    mx.launch_copy_strided(mx.COMPLEX64, mx.COMPLEX64, desc, Y.ptr, X.ptr)
    mx.sync()
    got = Y.download(np.complex64, n)
    assert np.array_equal(bits(got), bits(x.reshape(shape).transpose(perm).ravel()))


@pytest.mark.parametrize("src", list(NP))
def test_real_to_complex64(mx, orc, src):
    """A real dtype -> complex64 is (float(v), 0), strided source, against the oracle."""
    rng = np.random.default_rng(len(src) + 90)
    x = values(src, 2000, rng)
    desc = ([40, 25], [25, 1], [1, 40])              # a transposed source view
    X = mx.DeviceBuffer.from_numpy(x)
    Y = mx.DeviceBuffer(1000 * 8)
    mx.launch_copy_strided(mx.COMPLEX64, getattr(mx, src), desc, Y.ptr, X.ptr)
    mx.sync()
    got = Y.download(np.complex64, 1000)
    ref = orc.copy_strided(orc.C64, getattr(orc, orc_code(src)), [40, 25], [25, 1], [1, 40],
                           np.zeros(1000, np.complex64), x)
    g, r = got.view(np.float32), ref.view(np.float32)
    assert not ((bits(g) != bits(r)) & ~(np.isnan(g) & np.isnan(r))).any()


def test_complex64_to_real_is_rejected(mx):
    X = mx.DeviceBuffer(64)
    with pytest.raises(mx.MatrixAMDError):
        mx.launch_copy_strided(mx.FLOAT32, mx.COMPLEX64, ([4], [1], [1]), X.ptr, X.ptr)
