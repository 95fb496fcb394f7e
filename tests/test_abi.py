"""The C-ABI library loads and exports every entry point the public headers declare.

CPU-only: argument validation paths return before any HIP call, so they run without a GPU.
"""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

import matrix_amd as mx

ROOT = Path(__file__).resolve().parent.parent


def declared_symbols():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(mx_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_every_declared_symbol_is_exported():
    syms = declared_symbols()
    assert "mx_launch_bcast_binary" in syms and "mx_launch_reduce" in syms
    out = subprocess.run(["nm", "-D", "--defined-only", str(mx.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\bT (mx_[a-z0-9_]+)$", out, flags=re.M))
    missing = [s for s in syms if s not in exported]
    assert not missing, missing
    for s in syms:
        assert hasattr(mx.lib, s)


def test_library_is_gfx950_code_object():
    # the fat binary embedded in the library names its offload targets
    blob = open(mx.LIB_PATH, "rb").read()
    targets = set(re.findall(rb"amdgcn-amd-amdhsa--(gfx[0-9a-f]+)", blob))
    assert targets == {b"gfx950"}, targets


def test_invalid_arguments_fail_without_gpu():
    shape = mx.u32([4])
    st = mx.u32([1])
    rc = mx.lib.mx_launch_bcast_binary(99, mx.FLOAT32, 1, shape, st, st, st, 1, 1, 1, None)
    assert rc == mx.ERR_INVALID_ARG and "unknown op" in mx.last_error()
    rc = mx.lib.mx_launch_bcast_binary(0, mx.FLOAT32, 9, shape, st, st, st, 1, 1, 1, None)
    assert rc == mx.ERR_INVALID_ARG
    rc = mx.lib.mx_launch_reduce(7, mx.FLOAT32, 1, 4, 1, shape, st, st, 1, 1, None, 0, None)
    assert rc == mx.ERR_INVALID_ARG
    # zero elements: nothing to do, succeeds without touching a device
    zero = mx.u32([0])
    assert mx.lib.mx_launch_bcast_binary(0, mx.FLOAT32, 1, zero, st, st, st, None, None, None, None) == mx.OK


def test_unsupported_dtype_and_uninitialized_runtime():
    shape = mx.u32([4])
    st = mx.u32([1])
    # complex64 has no Max kernel (the reference instantiates Add / Sub / Mul / Divide only)
    rc = mx.lib.mx_launch_bcast_binary(mx.OP_MAX, mx.COMPLEX64, 1, shape, st, st, st, 8, 8, 8, ctypes.c_void_p(1))
    assert rc in (mx.ERR_UNSUPPORTED, mx.ERR_NOT_INITIALIZED)
    p = ctypes.c_void_p()
    if not mx._initialized:
        assert mx.lib.mx_hip_alloc(16, ctypes.byref(p)) == mx.ERR_NOT_INITIALIZED


def test_workspace_query_is_pure_host():
    # 4 rows of 2^20 are too few outputs for the CUs: each row is split -> partials + counters
    nb = mx.reduce_workspace_bytes(mx.RED_SUM, mx.FLOAT32, 1, 1 << 20, ([4], [1], [1 << 20]))
    assert nb > 0
    # 256 rows of 65536 take one block per row: no workspace
    assert mx.reduce_workspace_bytes(mx.RED_SUM, mx.FLOAT32, 1, 65536, ([256], [1], [65536])) == 0
    # add+row-sum's [4096, 1024] needs none
    assert mx.reduce_workspace_bytes(mx.RED_SUM, mx.FLOAT32, 1, 1024, ([4096], [1], [1024])) == 0
