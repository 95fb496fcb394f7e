"""The .npz boundary: matrix::save_as_npz (Matrix.mm:3748-4085) and matrix::load_npz.

oracle/npz.py restates the reference's writer; it is pinned here against zlib's CRC-32, the
CRC-32 check value, Python's zipfile (structure and CRCs) and numpy's np.load.  The C++ writer
(driven by tests/cpp/npz_test.cpp) must then produce the oracle's bytes exactly, and the C++
loader must read back both its own archives and numpy's np.savez files (ZIP64 local headers,
named entries, Fortran order).
"""
import io
import subprocess
import zipfile
import zlib
from pathlib import Path

import numpy as np
import pytest

from oracle import npz as onpz

ROOT = Path(__file__).resolve().parent.parent
BIN = ROOT / "tests" / "cpp" / "_build" / "npz_test"

NP_OF = {onpz.F32: np.float32, onpz.F16: np.float16, onpz.U8: np.uint8, onpz.I32: np.int32, onpz.I16: np.int16,
         onpz.U32: np.uint32, onpz.U16: np.uint16, onpz.BOOL: np.bool_, onpz.I8: np.int8, onpz.C64: np.complex64,
         onpz.I64: np.int64, onpz.U64: np.uint64}
# the entries npz_test.cpp `write` builds
CODES = [onpz.F32, onpz.F16, onpz.U8, onpz.I32, onpz.I16, onpz.U32, onpz.U16, onpz.BOOL, onpz.I8, onpz.C64,
         onpz.I64, onpz.U64]
SHAPES = [[3, 4], [5], [], [2, 3, 4], [2, 0, 3], [7, 1], [1, 2, 1, 3], [6], [4, 4], [3, 2], [2, 2, 2], [9]]


def ensure_built():
    if not BIN.exists():
        import importlib.util
        spec = importlib.util.spec_from_file_location("_mx_build", ROOT / "matrix_amd" / "build.py")
        b = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(b)
        b.build_test_programs()
    return BIN


def pattern(code, shape, i):
    n = int(np.prod(shape)) if shape else 1
    nb = n * np.dtype(NP_OF[code]).itemsize
    k = np.arange(nb, dtype=np.uint64)
    b = ((131 * k + 17 * i + 7) & 0xFF).astype(np.uint8)
    if code == onpz.BOOL:
        b &= 1
    return b.tobytes()


def pattern_entries():
    ent = [(c, s, pattern(c, s, i)) for i, (c, s) in enumerate(zip(CODES, SHAPES))]
    base = np.frombuffer(pattern(onpz.I32, [3, 5], 12), np.int32).reshape(3, 5)
    ent.append((onpz.I32, [5, 3], np.ascontiguousarray(base.T).tobytes()))
    return ent


def run(*args, timeout=120):
    return subprocess.run([str(ensure_built()), *map(str, args)], capture_output=True, text=True, timeout=timeout)


# ------------------------------------------------------------------ the oracle, pinned
def test_oracle_crc32_matches_zlib():
    assert onpz.crc32(b"123456789") == 0xCBF43926            # the CRC-32 check value
    rng = np.random.default_rng(0)
    for n in (0, 1, 7, 64, 1000):
        d = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert onpz.crc32(d) == zlib.crc32(d)


def test_oracle_archive_reads_back_with_numpy_and_zipfile():
    ent = pattern_entries()
    blob = onpz.save_as_npz(ent)
    zf = zipfile.ZipFile(io.BytesIO(blob))
    assert zf.testzip() is None                                   # every CRC-32 checks
    assert zf.namelist() == ["arr_%d.npy" % i for i in range(len(ent))]
    assert all(zi.compress_type == zipfile.ZIP_STORED for zi in zf.infolist())
    with np.load(io.BytesIO(blob)) as f:
        for i, (code, shape, data) in enumerate(ent):
            a = f["arr_%d" % i]
            assert a.dtype == np.dtype(NP_OF[code]) and list(a.shape) == shape
            assert a.tobytes() == data
    for i in range(len(ent)):                                     # header + data start on 64 bytes
        raw = zf.read("arr_%d.npy" % i)
        hl = int.from_bytes(raw[8:10], "little")
        assert (10 + hl) % 64 == 0 and raw[10 + hl - 1:10 + hl] == b"\n"


def test_oracle_shape_strings():
    assert onpz.shape_tuple([]) == "()"
    assert onpz.shape_tuple([5]) == "(5,)"
    assert onpz.shape_tuple([3, 4]) == "(3,4)"
    with pytest.raises(ValueError):
        onpz.npy_blob(onpz.BF16, [2], b"\0" * 4)


# ------------------------------------------------------------------ the C++ writer and loader
def test_writer_matches_oracle_bytes(tmp_path):
    out = tmp_path / "w.npz"
    r = run("write", out)
    assert r.returncode == 0, r.stderr
    assert out.read_bytes() == onpz.save_as_npz(pattern_entries())


def test_writer_rejects_bfloat16(tmp_path):
    r = run("bf16", tmp_path / "b.npz")
    assert r.returncode == 0 and "BFloat16" in r.stdout, r.stdout + r.stderr
    assert not (tmp_path / "b.npz").exists()


def test_loader_round_trips_own_archive(tmp_path):
    src, dst = tmp_path / "a.npz", tmp_path / "b.npz"
    src.write_bytes(onpz.save_as_npz(pattern_entries()))
    r = run("resave", src, dst)
    assert r.returncode == 0, r.stderr
    assert dst.read_bytes() == src.read_bytes()
    names = [ln.split()[0] for ln in r.stdout.splitlines()]
    assert names == ["arr_%d" % i for i in range(13)]


def test_loader_reads_numpy_savez(tmp_path):
    """np.savez writes ZIP64 fields into its local headers; named entries keep their order;
    a Fortran-ordered array loads with its values in place; the archive written back holds the
    same arrays (as arr_<i>)."""
    rng = np.random.default_rng(3)
    arrays = {
        "weights": rng.standard_normal([17, 9]).astype(np.float32),
        "ids": rng.integers(-2**62, 2**62, [11], dtype=np.int64),
        "mask": rng.integers(0, 2, [4, 6]).astype(np.bool_),
        "zs": (rng.standard_normal([5, 2]) + 1j * rng.standard_normal([5, 2])).astype(np.complex64),
        "half": rng.standard_normal([3, 3, 3]).astype(np.float16),
        "fort": np.asfortranarray(rng.standard_normal([6, 5, 4]).astype(np.float32)),
        "scalar": np.array(7, np.uint16),
    }
    src, dst = tmp_path / "np.npz", tmp_path / "back.npz"
    np.savez(src, **arrays)
    r = run("resave", src, dst)
    assert r.returncode == 0, r.stderr
    assert [ln.split()[0] for ln in r.stdout.splitlines()] == list(arrays)
    with np.load(dst) as f:
        for i, (k, v) in enumerate(arrays.items()):
            got = f["arr_%d" % i]
            assert got.dtype == v.dtype and got.shape == v.shape, k
            assert got.tobytes() == np.ascontiguousarray(v).tobytes(), k


def test_loader_errors(tmp_path):
    p = tmp_path / "c.npz"
    np.savez_compressed(p, a=np.arange(1000, dtype=np.float32))
    r = run("load", p)
    assert r.returncode == 3 and "compressed" in r.stdout, r.stdout + r.stderr
    blob = bytearray(onpz.save_as_npz([(onpz.F32, [4], np.arange(4, dtype=np.float32).tobytes())]))
    blob[100] ^= 0x01                                            # a data byte: the CRC-32 no longer matches
    p.write_bytes(bytes(blob))
    r = run("load", p)
    assert r.returncode == 3 and "CRC-32" in r.stdout, r.stdout + r.stderr
    p.write_bytes(b"not a zip file at all, just some bytes")
    r = run("load", p)
    assert r.returncode == 3, r.stdout + r.stderr


@pytest.mark.gpu
def test_device_results_round_trip(tmp_path):
    """Leaves loaded from np.savez, the sum, product and difference computed on the GPU and a
    transposed view of a device result, written by save_as_npz: equal to numpy's float32
    arithmetic (one correctly rounded operation each), and byte for byte the oracle's archive of
    those values."""
    rng = np.random.default_rng(5)
    a = rng.standard_normal([33, 70]).astype(np.float32)
    b = rng.standard_normal([33, 70]).astype(np.float32)
    src, dst = tmp_path / "in.npz", tmp_path / "out.npz"
    np.savez(src, a=a, b=b)
    r = run("gpu", src, dst, timeout=110)
    assert r.returncode == 0, r.stdout + r.stderr
    want = [a + b, a * b, np.ascontiguousarray((a + b).T), b - a]
    with np.load(dst) as f:
        for i, w in enumerate(want):
            assert np.array_equal(f["arr_%d" % i].view(np.uint32), w.view(np.uint32)), i
    ent = [(onpz.F32, list(w.shape), w.tobytes()) for w in want]
    assert dst.read_bytes() == onpz.save_as_npz(ent)
