"""matrix_amd -- MI355X (gfx950) evaluation path of the `matrix` lazy tensor library.

This package is a thin ctypes view of the C launch ABI (include/matrix_amd.h) and of the host
shape helpers (include/matrix_amd_shape.h), both exported by the in-tree library
`matrix_amd/_lib/libmatrix_amd.so`.  There is no fallback: importing fails if the library
has not been built (`python -m matrix_amd.build`).
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

_PKG = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("MATRIX_AMD_LIB", _PKG / "_lib" / "libmatrix_amd.so"))

if not LIB_PATH.exists():
    raise ImportError(
        f"matrix_amd: native library {LIB_PATH} is missing; build it with `python -m matrix_amd.build`"
    )

lib = ctypes.CDLL(str(LIB_PATH))

# ------------------------------------------------------------------ codes (include/matrix_amd.h)
OK, ERR_INVALID_ARG, ERR_UNSUPPORTED, ERR_HIP, ERR_NOT_INITIALIZED, ERR_WORKSPACE = range(6)

FLOAT32, FLOAT16, UINT8, INT32, INT16, UINT32, UINT16, BOOL, INT8, COMPLEX64, BFLOAT16, INT64, UINT64 = range(13)
OP_ADD, OP_SUB, OP_MUL, OP_DIV, OP_MAX, OP_MIN, OP_EQ = range(7)
RED_SUM, RED_MAX, RED_MIN, RED_ARGMAX, RED_ARGMIN = range(5)
REDUCE_GROUP_MAX = 8
MAX_DIMS = 8

# numpy storage dtype of every element code (16-bit floats stored as raw bits for bfloat16)
NP_DTYPE = {
    FLOAT32: np.float32, FLOAT16: np.float16, UINT8: np.uint8, INT32: np.int32, INT16: np.int16,
    UINT32: np.uint32, UINT16: np.uint16, BOOL: np.bool_, INT8: np.int8, BFLOAT16: np.uint16,
    INT64: np.int64, UINT64: np.uint64, COMPLEX64: np.complex64,
}
DTYPE_NAME = {
    FLOAT32: "f32", FLOAT16: "f16", UINT8: "u8", INT32: "i32", INT16: "i16", UINT32: "u32",
    UINT16: "u16", BOOL: "bool", INT8: "i8", BFLOAT16: "bf16", INT64: "i64", UINT64: "u64",
    COMPLEX64: "c64",
}


class MatrixAMDError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"[mx status {status}] {message}")
        self.status = status


_u32p = ctypes.POINTER(ctypes.c_uint32)
_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_i = ctypes.c_int
_u32 = ctypes.c_uint32
_u64 = ctypes.c_uint64
_ip = ctypes.POINTER(ctypes.c_int)

_SIGS = {
    "mx_last_error": ([], ctypes.c_char_p),
    "mx_version": ([], ctypes.c_char_p),
    "mx_hip_init": ([_i], _i),
    "mx_hip_shutdown": ([], _i),
    "mx_hip_device_count": ([_ip], _i),
    "mx_hip_alloc": ([_sz, ctypes.POINTER(_vp)], _i),
    "mx_hip_free": ([_vp], _i),
    "mx_hip_alloc_stats": ([ctypes.POINTER(_u64), ctypes.POINTER(_u64)], _i),
    "mx_hip_h2d": ([_vp, _vp, _sz, _vp], _i),
    "mx_hip_d2h": ([_vp, _vp, _sz, _vp], _i),
    "mx_hip_d2d": ([_vp, _vp, _sz, _vp], _i),
    "mx_hip_memset": ([_vp, _i, _sz, _vp], _i),
    "mx_hip_stream_for_thread": ([ctypes.POINTER(_vp)], _i),
    "mx_hip_sync": ([_vp], _i),
    "mx_hip_stream_create": ([ctypes.POINTER(_vp)], _i),
    "mx_hip_stream_destroy": ([_vp], _i),
    "mx_hip_stream_wait_event": ([_vp, _vp], _i),
    "mx_hip_event_create": ([ctypes.POINTER(_vp)], _i),
    "mx_hip_event_destroy": ([_vp], _i),
    "mx_hip_event_record": ([_vp, _vp], _i),
    "mx_hip_event_elapsed_ms": ([_vp, _vp, ctypes.POINTER(ctypes.c_float)], _i),
    "mx_launch_bcast_binary": ([_i, _i, _i, _u32p, _u32p, _u32p, _u32p, _vp, _vp, _vp, _vp], _i),
    "mx_reduce_workspace_bytes": ([_i, _i, _u32, _u32, _i, _u32p, _u32p, _u32p, ctypes.POINTER(_sz)], _i),
    "mx_launch_reduce": ([_i, _i, _u32, _u32, _i, _u32p, _u32p, _u32p, _vp, _vp, _vp, _sz, _vp], _i),
    "mx_launch_reduce_noalloc": ([_i, _i, _u32, _u32, _i, _u32p, _u32p, _u32p, _vp, _vp, _vp], _i),
    "mx_launch_reduce_group": ([_i, _ip, _i, _u32, _u32, _i, _u32p, _u32p, _u32p, ctypes.POINTER(_vp),
                                ctypes.POINTER(_vp), ctypes.POINTER(_vp), ctypes.POINTER(_sz), _vp], _i),
    "mx_collapse_dims3": ([_u32p, _u32p, _u32p, _u32p, _u32, _u64, _u32p, _u32p, _u32p, _u32p, _u32p], _i),
    "mx_collapse_dims2": ([_u32p, _u32p, _u32p, _u32, _u64, _u32p, _u32p, _u32p, _u32p], _i),
    "mx_collapse_dims_matmul": ([_u32p, _u32p, _u32p, _u32p, _u32, _u64, _u32p, _u32p, _u32p, _u32p, _u32p], _i),
    "mx_collapse_dims_reduce2": ([_u32p, _u32p, _u32p, _u32, _i, _i, _i, _u64, _u32p, _u32p, _u32p, _u32p], _i),
    "mx_broadcast_shapes": ([_u32p, _u32p, _u32, _u32p, _u32p, _u32, _u32p, _u32p, _u32p, _u32p, _u32p, _u32p], _i),
    "mx_broadcast_shapes_matmul": ([_u32p, _u32p, _u32, _u32p, _u32p, _u32, _u32p, _u32p, _u32p, _u32p, _u32p, _u32p], _i),
    "mx_launch_batched_matmul": ([_i, _i, _u32p, _u32p, _u32p, _u32p, _u32, _vp, _vp, _vp, _vp], _i),
    "mx_matmul_workspace_bytes": ([_i, _i, _u32p, _u32p, _u32p, _u32p, _u32, ctypes.POINTER(_sz)], _i),
    "mx_launch_batched_matmul_ws": ([_i, _i, _u32p, _u32p, _u32p, _u32p, _u32, _vp, _vp, _vp, _vp, _sz, _vp], _i),
    "mx_launch_max_grad": ([_i, _i, _i, _i, _u32p, _u32p, _u32p, _u32p, _vp, _vp, _vp, _vp, _vp], _i),
    "mx_launch_batched_matmul_bias_act": ([_i, _i, _u32p, _u32p, _u32p, _u32p, _u32, _vp, _vp, _vp, _vp, _vp, _i,
                                           _vp, _vp, _vp, _sz, _vp], _i),
    "mx_conv_workspace_bytes": ([_i, _i, _u32p, _u32p, _u32p, _u32p, _u32p, _u32p, _i, ctypes.POINTER(_sz)], _i),
    "mx_launch_conv_nd": ([_i, _i, _u32p, _u32p, _u32p, _u32p, _u32p, _u32p, _ip, _ip, _ip, _ip,
                           _i, _i, _vp, _vp, _vp, _vp, _sz, _vp], _i),
    "mx_launch_copy_strided": ([_i, _i, _i, _u32p, _u32p, _u32p, _vp, _vp, _vp], _i),
    "mx_launch_bcast_binary_reduce_rows": ([_i, _i, _i, _i, _u32p, _u32p, _u32p, _u32p, _u32, _vp, _vp, _vp, _vp,
                                            _vp], _i),
}

for _name, (_args, _res) in _SIGS.items():
    _f = getattr(lib, _name)
    _f.argtypes = _args
    _f.restype = _res


def last_error() -> str:
    msg = lib.mx_last_error()
    return msg.decode() if msg else ""


def check(status: int) -> None:
    if status != OK:
        raise MatrixAMDError(status, last_error())


def u32(seq) -> ctypes.Array:
    """uint32 ctypes array (at least one slot so a pointer is always valid)."""
    vals = [int(v) for v in seq]
    arr = (ctypes.c_uint32 * max(1, len(vals)))(*vals)
    return arr


def i32(seq) -> ctypes.Array:
    vals = [int(v) for v in seq]
    return (ctypes.c_int * max(1, len(vals)))(*vals)


# ------------------------------------------------------------------ device runtime
_initialized = False


def init(device: int = 0) -> None:
    global _initialized
    if not _initialized:
        check(lib.mx_hip_init(device))
        _initialized = True


def sync(stream=None) -> None:
    check(lib.mx_hip_sync(stream))


def device_count() -> int:
    n = ctypes.c_int(0)
    check(lib.mx_hip_device_count(ctypes.byref(n)))
    return n.value


class DeviceBuffer:
    """An owned device allocation (mx_hip_alloc / mx_hip_free)."""

    def __init__(self, nbytes: int):
        init()
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(lib.mx_hip_alloc(self.nbytes, ctypes.byref(p)))
        self.ptr = p.value or 0

    @classmethod
    def from_numpy(cls, arr: np.ndarray) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.nbytes)
        if arr.nbytes:
            check(lib.mx_hip_h2d(buf.ptr, arr.ctypes.data, arr.nbytes, None))
        return buf

    def upload(self, arr: np.ndarray, offset: int = 0) -> None:
        arr = np.ascontiguousarray(arr)
        assert offset + arr.nbytes <= self.nbytes
        if arr.nbytes:
            check(lib.mx_hip_h2d(self.ptr + offset, arr.ctypes.data, arr.nbytes, None))

    def download(self, dtype, count: int | None = None, offset: int = 0) -> np.ndarray:
        dt = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dt.itemsize
        out = np.empty(count, dtype=dt)
        if out.nbytes:
            assert offset + out.nbytes <= self.nbytes
            check(lib.mx_hip_d2h(out.ctypes.data, self.ptr + offset, out.nbytes, None))
        return out

    def fill_bytes(self, value: int) -> None:
        check(lib.mx_hip_memset(self.ptr, value, self.nbytes, None))

    def free(self) -> None:
        if self.ptr:
            lib.mx_hip_free(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    """An extra stream (mx_hip_stream_create); pass .ptr as a launch's stream."""

    def __init__(self):
        init()
        p = ctypes.c_void_p()
        check(lib.mx_hip_stream_create(ctypes.byref(p)))
        self.ptr = p.value

    def wait(self, event: "Event") -> None:
        check(lib.mx_hip_stream_wait_event(self.ptr, event.ptr))

    def sync(self) -> None:
        check(lib.mx_hip_sync(self.ptr))

    def __del__(self):
        try:
            lib.mx_hip_stream_destroy(self.ptr)
        except Exception:
            pass


def wait_event(event: "Event", stream=None) -> None:
    """Make `stream` (default: the calling thread's stream) wait for `event`."""
    check(lib.mx_hip_stream_wait_event(stream, event.ptr))


class Event:
    def __init__(self):
        p = ctypes.c_void_p()
        check(lib.mx_hip_event_create(ctypes.byref(p)))
        self.ptr = p.value

    def record(self, stream=None) -> None:
        check(lib.mx_hip_event_record(self.ptr, stream))

    def elapsed_ms(self, later: "Event") -> float:
        ms = ctypes.c_float()
        check(lib.mx_hip_event_elapsed_ms(self.ptr, later.ptr, ctypes.byref(ms)))
        return ms.value

    def __del__(self):
        try:
            lib.mx_hip_event_destroy(self.ptr)
        except Exception:
            pass


# ------------------------------------------------------------------ host shape helpers
def _out_arrays(n=4):
    return [(ctypes.c_uint32 * MAX_DIMS)() for _ in range(n)]


def collapse_dims3(shape, sA, sB, sC, size_cap=2**31 - 1):
    o = _out_arrays(4)
    nd = ctypes.c_uint32()
    check(lib.mx_collapse_dims3(u32(shape), u32(sA), u32(sB), u32(sC), len(shape), size_cap, *o, ctypes.byref(nd)))
    n = nd.value
    return [list(a[:n]) for a in o]


def collapse_dims2(shape, sA, sB, size_cap=2**31 - 1):
    o = _out_arrays(3)
    nd = ctypes.c_uint32()
    check(lib.mx_collapse_dims2(u32(shape), u32(sA), u32(sB), len(shape), size_cap, *o, ctypes.byref(nd)))
    n = nd.value
    return [list(a[:n]) for a in o]


def collapse_dims_matmul(shape, sA, sB, sC, size_cap=2**31 - 1):
    o = _out_arrays(4)
    nd = ctypes.c_uint32()
    check(lib.mx_collapse_dims_matmul(u32(shape), u32(sA), u32(sB), u32(sC), len(shape), size_cap, *o,
                                      ctypes.byref(nd)))
    n = nd.value
    return [list(a[:n]) for a in o]


def collapse_dims_reduce2(shape, sOut, sIn, axis, keep_dims=False, outer_collapsed=True, size_cap=2**32 - 1):
    o = _out_arrays(3)
    nd = ctypes.c_uint32()
    check(lib.mx_collapse_dims_reduce2(u32(shape), u32(sOut), u32(sIn), len(shape), axis, int(keep_dims),
                                       int(outer_collapsed), size_cap, *o, ctypes.byref(nd)))
    n = nd.value
    return [list(a[:n]) for a in o]


def broadcast_shapes(shape1, strides1, shape2, strides2, matmul=False):
    o = _out_arrays(6)
    fn = lib.mx_broadcast_shapes_matmul if matmul else lib.mx_broadcast_shapes
    check(fn(u32(shape1), u32(strides1), len(shape1), u32(shape2), u32(strides2), len(shape2), *o))
    n = max(len(shape1), len(shape2))
    return [list(a[:n]) for a in o]


def contiguous_strides(shape):
    st, acc = [0] * len(shape), 1
    for i in range(len(shape) - 1, -1, -1):
        st[i] = acc
        acc *= int(shape[i])
    return st


# ------------------------------------------------------------------ kernel launches
def launch_bcast_binary(op, dtype, desc, R, A, B, stream=None):
    shape, sA, sB, sR = desc
    check(lib.mx_launch_bcast_binary(op, dtype, len(shape), u32(shape), u32(sR), u32(sA), u32(sB),
                                     int(R), int(A), int(B), stream))


def reduce_workspace_bytes(op, dtype, reduce_stride, n_reduce, desc):
    shape, sOut, sIn = desc
    nb = ctypes.c_size_t()
    check(lib.mx_reduce_workspace_bytes(op, dtype, reduce_stride, n_reduce, len(shape), u32(shape), u32(sOut),
                                        u32(sIn), ctypes.byref(nb)))
    return nb.value


def matmul_workspace_bytes(dtype, desc, K):
    """Split-K workspace bytes of a product (mx_matmul_workspace_bytes); 0 when it never splits."""
    shape, sA, sBt, sC = desc
    nb = ctypes.c_size_t()
    check(lib.mx_matmul_workspace_bytes(dtype, len(shape), u32(shape), u32(sA), u32(sBt), u32(sC), K,
                                        ctypes.byref(nb)))
    return nb.value


def launch_batched_matmul(dtype, desc, K, C, A, Bt, stream=None, workspace=0, workspace_bytes=0):
    """desc = (shapeC [..., M, N], sA, sBt, sC) as collapse_dims_matmul gives it.  With a workspace
    (mx_launch_batched_matmul_ws) the K range may be split over blocks; without one the
    reference-signature entry point runs the product unsplit."""
    shape, sA, sBt, sC = desc
    if workspace:
        check(lib.mx_launch_batched_matmul_ws(dtype, len(shape), u32(shape), u32(sA), u32(sBt), u32(sC), K,
                                              int(C), int(A), int(Bt), int(workspace), workspace_bytes, stream))
    else:
        check(lib.mx_launch_batched_matmul(dtype, len(shape), u32(shape), u32(sA), u32(sBt), u32(sC), K,
                                           int(C), int(A), int(Bt), stream))


def alloc_stats():
    """(allocations, frees) of device memory made through the ABI so far."""
    a, f = ctypes.c_uint64(), ctypes.c_uint64()
    check(lib.mx_hip_alloc_stats(ctypes.byref(a), ctypes.byref(f)))
    return a.value, f.value


def launch_max_grad(op, side, dtype, desc, R, A, B, G, stream=None):
    """Gradient of Max / Min (op) to operand a (side 0) or b (side 1): desc as for
    launch_bcast_binary, G read with R's strides."""
    shape, sA, sB, sR = desc
    check(lib.mx_launch_max_grad(op, side, dtype, len(shape), u32(shape), u32(sR), u32(sA), u32(sB), int(R), int(A),
                                 int(B), int(G), stream))


def launch_batched_matmul_bias_act(dtype, desc, K, C, A, Bt, bias, Z, act_op, act_scalar, H, stream=None,
                                   workspace=0, workspace_bytes=0):
    """C = A . Bt^T, Z = C + bias (N elements), H = act_op(Z, *act_scalar) (OP_MAX / OP_MIN) in one
    call; desc and workspace as for launch_batched_matmul, C / Z / H contiguous."""
    shape, sA, sBt, sC = desc
    check(lib.mx_launch_batched_matmul_bias_act(dtype, len(shape), u32(shape), u32(sA), u32(sBt), u32(sC), K,
                                                int(C), int(A), int(Bt), int(bias), int(Z), act_op,
                                                int(act_scalar), int(H), int(workspace), workspace_bytes, stream))


def launch_reduce(op, dtype, reduce_stride, n_reduce, desc, out, inp, workspace=0, workspace_bytes=0,
                  stream=None):
    shape, sOut, sIn = desc
    check(lib.mx_launch_reduce(op, dtype, reduce_stride, n_reduce, len(shape), u32(shape), u32(sOut), u32(sIn),
                               int(out), int(inp), int(workspace), workspace_bytes, stream))


REDUCE_NOALLOC_SCRATCH_BYTES = 4 << 20


def launch_reduce_noalloc(op, dtype, reduce_stride, n_reduce, desc, out, inp, stream=None):
    """mx_launch_reduce_noalloc: launch_reduce without a workspace (split partials in the
    library's fixed per-GPU scratch; calls on one GPU must not overlap in time)."""
    shape, sOut, sIn = desc
    check(lib.mx_launch_reduce_noalloc(op, dtype, reduce_stride, n_reduce, len(shape), u32(shape), u32(sOut),
                                       u32(sIn), int(out), int(inp), stream))


def _group_arrays(ops, outs, ins, workspaces, workspace_bytes):
    n = len(ops)
    if not (len(outs) == len(ins) == n):
        raise ValueError("reduce group: ops, outs and ins differ in length")
    workspaces = list(workspaces) if workspaces is not None else [0] * n
    workspace_bytes = list(workspace_bytes) if workspace_bytes is not None else [0] * n
    return (n, (ctypes.c_int * n)(*ops), (_vp * n)(*[int(o) for o in outs]), (_vp * n)(*[int(i) for i in ins]),
            (_vp * n)(*[int(w) for w in workspaces]), (_sz * n)(*workspace_bytes))


def launch_reduce_group(ops, dtype, reduce_stride, n_reduce, desc, outs, ins, workspaces=None, workspace_bytes=None,
                        stream=None):
    """mx_launch_reduce_group: member k reduces ins[k] with ops[k] into outs[k] (one descriptor)."""
    shape, sOut, sIn = desc
    n, o, po, pi, pw, pb = _group_arrays(ops, outs, ins, workspaces, workspace_bytes)
    check(lib.mx_launch_reduce_group(n, o, dtype, reduce_stride, n_reduce, len(shape), u32(shape), u32(sOut), u32(sIn),
                                     po, pi, pw, pb, stream))


def prepare_reduce_group(ops, dtype, reduce_stride, n_reduce, desc, workspaces=None, workspace_bytes=None,
                         stream=None):
    """mx_launch_reduce_group with its descriptor and ops converted once: returns launch(outs, ins)."""
    shape, sOut, sIn = desc
    n = len(ops)
    fn = lib.mx_launch_reduce_group
    opa = (ctypes.c_int * n)(*ops)
    pw = (_vp * n)(*[int(w) for w in (workspaces or [0] * n)])
    pb = (_sz * n)(*(workspace_bytes or [0] * n))
    head = (dtype, reduce_stride, n_reduce, len(shape), u32(shape), u32(sOut), u32(sIn))
    po, pi = (_vp * n)(), (_vp * n)()

    def launch(outs, ins):
        for k in range(n):
            po[k], pi[k] = int(outs[k]), int(ins[k])
        status = fn(n, opa, *head, po, pi, pw, pb, stream)
        if status != OK:
            raise MatrixAMDError(status, last_error())

    return launch


def launch_bcast_binary_reduce_rows(op, red_op, dtype, desc, n, R, A, B, out, stream=None):
    """R = A op B (desc as for launch_bcast_binary) and out[r] = red_op over R's rows of n."""
    shape, sA, sB, sR = desc
    check(lib.mx_launch_bcast_binary_reduce_rows(op, red_op, dtype, len(shape), u32(shape), u32(sR), u32(sA),
                                                 u32(sB), n, int(R), int(A), int(B), int(out), stream))


def prepare_bcast_binary_reduce_rows(op, red_op, dtype, desc, n, stream=None):
    """launch_bcast_binary_reduce_rows with its descriptor converted once: returns launch(R, A, B, out)."""
    shape, sA, sB, sR = desc
    fn = lib.mx_launch_bcast_binary_reduce_rows
    head = (op, red_op, dtype, len(shape), u32(shape), u32(sR), u32(sA), u32(sB), n)

    def launch(R, A, B, out):
        status = fn(*head, R, A, B, out, stream)
        if status != OK:
            raise MatrixAMDError(status, last_error())

    return launch


def prepare_bcast_binary(op, dtype, desc, stream=None):
    """mx_launch_bcast_binary with its descriptor converted once: returns launch(R, A, B)."""
    shape, sA, sB, sR = desc
    fn = lib.mx_launch_bcast_binary
    head = (op, dtype, len(shape), u32(shape), u32(sR), u32(sA), u32(sB))

    def launch(R, A, B):
        status = fn(*head, R, A, B, stream)
        if status != OK:
            raise MatrixAMDError(status, last_error())

    return launch


def prepare_reduce(op, dtype, reduce_stride, n_reduce, desc, workspace=0, workspace_bytes=0, stream=None):
    """mx_launch_reduce with its descriptor converted once: returns launch(out, inp) for launches
    repeated many times (a compiled graph node's execute)."""
    shape, sOut, sIn = desc
    fn = lib.mx_launch_reduce
    head = (op, dtype, reduce_stride, n_reduce, len(shape), u32(shape), u32(sOut), u32(sIn))
    tail = (int(workspace), workspace_bytes, stream)

    def launch(out, inp):
        status = fn(*head, out, inp, *tail)
        if status != OK:
            raise MatrixAMDError(status, last_error())

    return launch


def prepare_batched_matmul(dtype, desc, K, stream=None, workspace=0, workspace_bytes=0):
    """mx_launch_batched_matmul_ws with its descriptor converted once: returns launch(C, A, Bt)."""
    shape, sA, sBt, sC = desc
    fn = lib.mx_launch_batched_matmul_ws
    head = (dtype, len(shape), u32(shape), u32(sA), u32(sBt), u32(sC), K)
    tail = (int(workspace), workspace_bytes, stream)

    def launch(C, A, Bt):
        status = fn(*head, C, A, Bt, *tail)
        if status != OK:
            raise MatrixAMDError(status, last_error())

    return launch


def conv_workspace_bytes(dtype, geom):
    """geom = dict(in_shape, k_shape, out_shape, in_strides, k_strides, out_strides, groups, ...)."""
    nb = ctypes.c_size_t()
    ns = len(geom["in_shape"]) - 2
    check(lib.mx_conv_workspace_bytes(dtype, ns, u32(geom["in_shape"]), u32(geom["k_shape"]),
                                      u32(geom["out_shape"]), u32(geom["in_strides"]), u32(geom["k_strides"]),
                                      u32(geom["out_strides"]), int(geom.get("groups", 1)), ctypes.byref(nb)))
    return nb.value


def launch_conv_nd(dtype, geom, out, inp, kern, workspace=0, workspace_bytes=0, stream=None):
    """Channels-last N-D convolution (conv_gpu's argument set).  geom holds in_shape
    [N, S.., C], k_shape [O, K.., C/groups], out_shape [N, O.., O], the three stride lists,
    pad, stride, dil (kernel), dil_lhs (input), groups and flip; missing geometry defaults to
    pad 0, stride 1, dilation 1, groups 1, no flip."""
    ns = len(geom["in_shape"]) - 2
    pad = geom.get("pad", [0] * ns)
    stride = geom.get("stride", [1] * ns)
    dil = geom.get("dil", [1] * ns)
    dil_lhs = geom.get("dil_lhs", [1] * ns)
    check(lib.mx_launch_conv_nd(dtype, ns, u32(geom["in_shape"]), u32(geom["k_shape"]), u32(geom["out_shape"]),
                                u32(geom["in_strides"]), u32(geom["k_strides"]), u32(geom["out_strides"]),
                                i32(pad), i32(stride), i32(dil), i32(dil_lhs), int(geom.get("groups", 1)),
                                int(geom.get("flip", 0)), int(out), int(inp), int(kern), int(workspace),
                                workspace_bytes, stream))


def prepare_conv_nd(dtype, geom, workspace=0, workspace_bytes=0, stream=None):
    """mx_launch_conv_nd with its geometry converted once: returns launch(out, inp, kern)."""
    ns = len(geom["in_shape"]) - 2
    fn = lib.mx_launch_conv_nd
    head = (dtype, ns, u32(geom["in_shape"]), u32(geom["k_shape"]), u32(geom["out_shape"]),
            u32(geom["in_strides"]), u32(geom["k_strides"]), u32(geom["out_strides"]),
            i32(geom.get("pad", [0] * ns)), i32(geom.get("stride", [1] * ns)), i32(geom.get("dil", [1] * ns)),
            i32(geom.get("dil_lhs", [1] * ns)), int(geom.get("groups", 1)), int(geom.get("flip", 0)))
    tail = (int(workspace), workspace_bytes, stream)

    def launch(out, inp, kern):
        status = fn(*head, out, inp, kern, *tail)
        if status != OK:
            raise MatrixAMDError(status, last_error())

    return launch


def launch_copy_strided(dst_dtype, src_dtype, desc, dst, src, stream=None):
    """desc = (shape, sDst, sSrc) over a collapsed iteration space (empty shape: one element)."""
    shape, sDst, sSrc = desc
    check(lib.mx_launch_copy_strided(dst_dtype, src_dtype, len(shape), u32(shape), u32(sDst), u32(sSrc),
                                     int(dst), int(src), stream))
