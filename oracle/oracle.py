"""ctypes view of the CPU oracle (oracle/_build/liboracle.so).

TEST INFRASTRUCTURE ONLY: the restatement of the reference's CPU eval that the GPU path is
checked against.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
import this module; the product (matrix_amd/) never does.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "liboracle.so"

F32, F16, U8, I32, I16, U32, U16, BOOL, I8, C64, BF16, I64, U64 = range(13)
ADD, SUB, MUL, DIV, MAX, MIN, EQ = range(7)
RSUM, RMAX, RMIN, RARGMAX, RARGMIN = range(5)
ACC_LITERAL, ACC_F32 = 0, 1

NP_DTYPE = {
    F32: np.float32, F16: np.float16, U8: np.uint8, I32: np.int32, I16: np.int16, U32: np.uint32,
    U16: np.uint16, BOOL: np.bool_, I8: np.int8, BF16: np.uint16, I64: np.int64, U64: np.uint64,
    C64: np.complex64,
}

_lib = None


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(f"oracle library {LIB_PATH} missing; run `make -C oracle`")
        L = ctypes.CDLL(str(LIB_PATH))
        u32p = ctypes.POINTER(ctypes.c_uint32)
        ip = ctypes.POINTER(ctypes.c_int)
        vp, i, u32, u64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint32, ctypes.c_uint64
        L.orc_bcast_binary.argtypes = [i, i, i, u32p, u32p, u32p, u32p, u64, vp, vp, vp]
        L.orc_reduce.argtypes = [i, i, i, u32, u32, i, u32p, u32p, u32p, u64, vp, vp, i]
        L.orc_batched_matmul.argtypes = [i, i, i, u32p, u32p, u32p, u32p, u32, vp, vp, vp, i]
        L.orc_conv.argtypes = [i, i, i, u32p, u32p, u32p, u32p, u32p, u32p, ip, ip, ip, ip, i, i, vp, vp, vp, i]
        L.orc_copy_strided.argtypes = [i, i, i, u32p, u32p, u32p, u64, vp, vp]
        for f in ("orc_bcast_binary", "orc_reduce", "orc_batched_matmul", "orc_conv", "orc_copy_strided"):
            getattr(L, f).restype = i
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_f32_to_f16.argtypes = [ctypes.c_float]
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f32_to_bf16.argtypes = [ctypes.c_float]
        L.orc_f32_to_bf16.restype = ctypes.c_uint16
        L.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_bf16_to_f32.restype = ctypes.c_float
        L.orc_f16_to_f32_n.argtypes = [vp, vp, ctypes.c_size_t]
        L.orc_f32_to_f16_n.argtypes = [vp, vp, ctypes.c_size_t]
        L.orc_f32_to_bf16_n.argtypes = [vp, vp, ctypes.c_size_t]
        _lib = L
    return _lib


def _u32(seq):
    vals = [int(v) for v in seq]
    return (ctypes.c_uint32 * max(1, len(vals)))(*vals)


def _i32(seq):
    vals = [int(v) for v in seq]
    return (ctypes.c_int * max(1, len(vals)))(*vals)


def _ptr(a: np.ndarray):
    return a.ctypes.data


def default_threads() -> int:
    """OpenMP threads for parity runs (never the timed baseline): at most 16, the CPU share of
    one GPU on the GPU host."""
    return int(os.environ.get("ORACLE_THREADS", min(16, os.cpu_count() or 1)))


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    load().orc_f32_to_f16_n(_ptr(x), _ptr(out), x.size)
    return out


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    load().orc_f16_to_f32_n(_ptr(h), _ptr(out), h.size)
    return out


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    load().orc_f32_to_bf16_n(_ptr(x), _ptr(out), x.size)
    return out


def bcast_binary(op, dtype, desc, total, A: np.ndarray, B: np.ndarray, out_dtype=None) -> np.ndarray:
    """desc = (shape, sA, sB, sR) collapsed; returns the flat output of `total` elements."""
    shape, sA, sB, sR = desc
    R = np.zeros(max(total, 1), dtype=out_dtype or A.dtype)
    rc = load().orc_bcast_binary(op, dtype, len(shape), _u32(shape), _u32(sR), _u32(sA), _u32(sB), total,
                                 _ptr(R), _ptr(np.ascontiguousarray(A)), _ptr(np.ascontiguousarray(B)))
    if rc != 0:
        raise ValueError("orc_bcast_binary: unsupported op/dtype")
    return R[:total] if total else R[:0]


def reduce(op, dtype, reduce_stride, n_reduce, desc, total_out, X: np.ndarray, acc=ACC_F32,
           nthreads=None) -> np.ndarray:
    shape, sOut, sIn = desc
    out_dt = np.int32 if op in (RARGMAX, RARGMIN) else X.dtype
    out = np.zeros(max(total_out, 1), dtype=out_dt)
    rc = load().orc_reduce(op, dtype, acc, reduce_stride, n_reduce, len(shape), _u32(shape), _u32(sOut),
                           _u32(sIn), total_out, _ptr(out), _ptr(np.ascontiguousarray(X)),
                           nthreads or default_threads())
    if rc != 0:
        raise ValueError("orc_reduce: unsupported op/dtype")
    return out[:total_out]


def batched_matmul(dtype, desc, K, A: np.ndarray, Bt: np.ndarray, out_size: int, acc=ACC_F32,
                   nthreads=None) -> np.ndarray:
    shape, sA, sBt, sC = desc
    C = np.zeros(out_size, dtype=A.dtype)
    rc = load().orc_batched_matmul(dtype, acc, len(shape), _u32(shape), _u32(sA), _u32(sBt), _u32(sC), K,
                                   _ptr(C), _ptr(np.ascontiguousarray(A)), _ptr(np.ascontiguousarray(Bt)),
                                   nthreads or default_threads())
    if rc != 0:
        raise ValueError("orc_batched_matmul: unsupported dtype")
    return C


def conv(dtype, in_shape, k_shape, out_shape, in_strides, k_strides, out_strides, pad, stride, dil, dil_lhs,
         groups, flip, X: np.ndarray, W: np.ndarray, out_size: int, acc=ACC_F32, nthreads=None) -> np.ndarray:
    ns = len(in_shape) - 2
    out = np.zeros(out_size, dtype=X.dtype)
    rc = load().orc_conv(dtype, acc, ns, _u32(in_shape), _u32(k_shape), _u32(out_shape), _u32(in_strides),
                         _u32(k_strides), _u32(out_strides), _i32(pad), _i32(stride), _i32(dil), _i32(dil_lhs),
                         groups, int(flip), _ptr(out), _ptr(np.ascontiguousarray(X)),
                         _ptr(np.ascontiguousarray(W)), nthreads or default_threads())
    if rc != 0:
        raise ValueError("orc_conv: unsupported dtype")
    return out


def copy_strided(dst_dtype, src_dtype, shape, sDst, sSrc, dst: np.ndarray, src: np.ndarray) -> np.ndarray:
    total = int(np.prod(shape)) if len(shape) else 1
    rc = load().orc_copy_strided(dst_dtype, src_dtype, len(shape), _u32(shape), _u32(sDst), _u32(sSrc), total,
                                 _ptr(dst), _ptr(np.ascontiguousarray(src)))
    if rc != 0:
        raise ValueError("orc_copy_strided: unsupported dtype")
    return dst
