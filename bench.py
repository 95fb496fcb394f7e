#!/usr/bin/env python3
"""Throughput of the MI355X evaluation path on the reductions workload.

One step = every reduction of the workload on X[256, 65536] float32 (N(0,1), seed 0, 30% of
rows with duplicated extrema):
  Sum / Max / Min / ArgMax / ArgMin over axis 1 (long rows) and over axis 0 (strided columns),
  and on X.reshape(64, 4, 4096, 16): Sum / Max / Min over axis 3 then axis 1,
  ArgMax / ArgMin over axis 3 and over axis 1 separately.
`value` = algorithmic HBM bytes of the step (inputs read + outputs written) / step time, with
inputs resident in HBM and rotated over enough copies that the 256 MB Infinity Cache cannot
hold the working set.  The step is one execute of the workload's compiled graph through the C++
graph API (matrix_amd/_bin/reductions_step: build once, compile once, then execute +
clear_trace_checks per step, each execute ending in its stream wait, as execute_metal does).
The executor runs independent reductions with one collapsed descriptor as one group launch
(mx_launch_reduce_group: the five over axis 1, the five over axis 0, the five over axis 3 of the
reshape, the three chained over axis 1 after them, ArgMax / ArgMin over axis 1 of the reshape)
and the graph's independent parts on two streams.

Prints one JSON line.  `roofline` is the dominant kernel's bytes per launch over its average
duration: the group launch that takes longest, timed with HIP events on its launch stream over
back-to-back launches on rotated inputs.  `cpu_baseline` times the oracle (the reference's CPU
loops restated) single-threaded on a bounded sample on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
N_COPIES = 17         # one 64 MiB copy of X per reduction that reads it (1.1 GB > the 256 MB MALL)


def contiguous_strides(shape):
    st, acc = [0] * len(shape), 1
    for i in range(len(shape) - 1, -1, -1):
        st[i] = acc
        acc *= int(shape[i])
    return st


def make_input(seed=0):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal([256, 65536]).astype(np.float32)
    # 30% of rows: copy the row max to 1-3 more positions (tie-breaking stress)
    for r in np.nonzero(rng.random(256) < 0.3)[0]:
        x[r, rng.integers(0, 65536, rng.integers(1, 4))] = x[r].max()
    return x


def build_ops(mx):
    """List of (name, op, in_shape, axis, input_kind); input_kind 'X' or an intermediate key."""
    ops = []
    names = {mx.RED_SUM: "sum", mx.RED_MAX: "max", mx.RED_MIN: "min", mx.RED_ARGMAX: "argmax",
             mx.RED_ARGMIN: "argmin"}
    for axis in (1, 0):
        for op in (mx.RED_SUM, mx.RED_MAX, mx.RED_MIN, mx.RED_ARGMAX, mx.RED_ARGMIN):
            ops.append((f"{names[op]}_axis{axis}", op, [256, 65536], axis, "X"))
    for op in (mx.RED_SUM, mx.RED_MAX, mx.RED_MIN):
        ops.append((f"{names[op]}_r4_axis3", op, [64, 4, 4096, 16], 3, "X"))
        ops.append((f"{names[op]}_r4_axis3_axis1", op, [64, 4, 4096], 1, f"{names[op]}_r4_axis3"))
    for op in (mx.RED_ARGMAX, mx.RED_ARGMIN):
        ops.append((f"{names[op]}_r4_axis3", op, [64, 4, 4096, 16], 3, "X"))
        ops.append((f"{names[op]}_r4_axis1", op, [64, 4, 4096, 16], 1, "X"))
    return ops


class Prepared:
    def __init__(self, mx, name, op, shape, axis, src):
        self.name, self.op, self.shape, self.axis, self.src = name, op, shape, axis, src
        self.tag = name.split("_", 1)[1]                 # shape / axis part of the op name
        out_shape = [s for i, s in enumerate(shape) if i != axis]
        self.desc = mx.collapse_dims_reduce2(shape, contiguous_strides(out_shape), contiguous_strides(shape), axis)
        self.rs = contiguous_strides(shape)[axis]
        self.n = shape[axis]
        self.total = int(np.prod(out_shape))
        self.out_bytes = self.total * 4
        self.in_bytes = int(np.prod(shape)) * 4
        self.bytes = self.in_bytes + self.out_bytes
        self.ws = mx.reduce_workspace_bytes(op, mx.FLOAT32, self.rs, self.n, self.desc)
        self.W = mx.DeviceBuffer(self.ws) if self.ws else None
        self.O = mx.DeviceBuffer(self.out_bytes)
        self._launch = mx.prepare_reduce(op, mx.FLOAT32, self.rs, self.n, self.desc,
                                         self.W.ptr if self.W else 0, self.ws)

    def launch(self, mx, in_ptr):
        self._launch(self.O.ptr, in_ptr)


class PreparedGroup:
    """The reductions of one descriptor (same shape and axis) as one mx_launch_reduce_group launch,
    as the graph executor groups them."""

    def __init__(self, mx, members):
        self.members = members
        m0 = members[0]
        self.name = "group_" + m0.tag
        self.bytes = sum(p.bytes for p in members)
        self._launch = mx.prepare_reduce_group([p.op for p in members], mx.FLOAT32, m0.rs, m0.n, m0.desc,
                                               [p.W.ptr if p.W else 0 for p in members], [p.ws for p in members])

    def launch(self, ins):
        self._launch([p.O.ptr for p in self.members], ins)


def make_groups(mx, prepared):
    """Groups of up to 8 ops with one (shape, axis), in workload order."""
    groups, by_key = [], {}
    for j, p in enumerate(prepared):
        key = (tuple(p.shape), p.axis)
        if key not in by_key or len(by_key[key][-1]) >= mx.REDUCE_GROUP_MAX:
            by_key.setdefault(key, []).append([])
            groups.append(by_key[key][-1])
        by_key[key][-1].append(j)
    return groups


def run_gpu(args):
    import matrix_amd as mx
    mx.init(0)
    x = make_input(0)
    copies = [mx.DeviceBuffer.from_numpy(x) for _ in range(N_COPIES)]
    prepared = [Prepared(mx, *o) for o in build_ops(mx)]
    by_name = {p.name: p for p in prepared}
    groups = [(idx, PreparedGroup(mx, [prepared[j] for j in idx])) for idx in make_groups(mx, prepared)]

    # every op reading X has its own resident copy (its ordinal among the ops on X), so no read of
    # X in a step can be served by the Infinity Cache from an earlier read of the same step
    ordinal = {}
    for p in prepared:
        if p.src == "X":
            ordinal[p.name] = len(ordinal)
    assert len(ordinal) == N_COPIES

    def src_of(p, c):
        return copies[c % N_COPIES].ptr if p.src == "X" else by_name[p.src].O.ptr

    def step(i):
        # the step as the executor runs it: one launch per group (members in workload order)
        for idx, g in groups:
            g.launch([src_of(prepared[j], ordinal.get(prepared[j].name, 0)) for j in idx])

    for i in range(args.warmup):
        step(i)
    mx.sync()
    t0 = time.perf_counter()
    e0, e1 = mx.Event(), mx.Event()
    e0.record()
    for i in range(args.steps):
        step(i)
    e1.record()
    mx.sync()
    wall = time.perf_counter() - t0
    ms_step = e0.elapsed_ms(e1) / args.steps
    step_bytes = sum(p.bytes for p in prepared)

    # durations per group launch and per single-op launch (events bracket the launches on the
    # launch stream): consecutive launches take the next copies, so a copy is read again only
    # after N_COPIES - 1 other reads of X; a group's chained inputs are its producers' outputs
    reps = max(3, min(40, 2 * args.steps))
    per_group = {}
    for idx, g in groups:
        a, b = mx.Event(), mx.Event()
        a.record()
        for i in range(reps):
            g.launch([src_of(prepared[j], i * len(idx) + k) for k, j in enumerate(idx)])
        b.record()
        mx.sync()
        per_group[g.name] = (a.elapsed_ms(b) / reps, g)
    per_op = {}
    for p in prepared:
        # the first launch of a kernel loads its code object: keep it out of the timing
        p.launch(mx, src_of(p, 0))
        mx.sync()
        a, b = mx.Event(), mx.Event()
        a.record()
        for i in range(reps):
            p.launch(mx, src_of(p, i))
        b.record()
        mx.sync()
        per_op[p.name] = a.elapsed_ms(b) / reps
    dom_name, (dom_ms, dom) = max(per_group.items(), key=lambda kv: kv[1][0])
    achieved = dom.bytes / (dom_ms * 1e-3) / 1e9
    return {
        "ms_per_step": ms_step, "wall_s": wall, "step_bytes": step_bytes,
        "value": step_bytes / (ms_step * 1e-3) / 1e9,
        "dominant": dom_name, "dominant_bytes": dom.bytes, "dominant_ms": dom_ms,
        "dominant_members": [p.name for p in dom.members],
        "achieved": achieved,
        "per_group_gbs": {k: round(g.bytes / (ms * 1e-3) / 1e9, 1) for k, (ms, g) in per_group.items()},
        "per_op_gbs": {k: round(by_name[k].bytes / (v * 1e-3) / 1e9, 1) for k, v in per_op.items()},
        "cpu_ops": [(p.name, p.op, p.shape, p.axis, p.src, p.desc, p.rs, p.n, p.total, p.bytes) for p in prepared],
    }


MFMA_PEAK_TFLOPS = {"f32": 157.3, "f16": 2500.0}


def _timed(mx, fn, reps):
    """Average ms per call of fn over reps back-to-back calls (HIP events on the launch stream)."""
    fn()
    mx.sync()
    e0, e1 = mx.Event(), mx.Event()
    e0.record()
    for i in range(reps):
        fn(i)
    e1.record()
    mx.sync()
    return e0.elapsed_ms(e1) / reps


def _best(mx, fn, reps, runs=2):
    """The faster of `runs` _timed measurements (the first run after an idle spell can catch the
    GPU below its working clock)."""
    return min(_timed(mx, fn, reps) for _ in range(runs))


def _normal(rng, shape, scale, dt):
    x = (rng.standard_normal(shape, dtype=np.float32) * np.float32(scale))
    return x.astype(np.float16) if dt == "f16" else x


def config_add_rowsum(mx):
    """Config 1: C = A[4096,1024] + B[1,1024] (broadcast), s = C.sum(1); 20 rotated copies of A
    (320 MiB, more than the Infinity Cache).  The graph executor fuses the two nodes into one launch
    (C still written); GB/s and frac_hbm count the bytes that launch moves (33,574,912)."""
    rng = np.random.default_rng(0)
    a = rng.standard_normal([4096, 1024], dtype=np.float32)
    b = rng.uniform(-1, 1, [1, 1024]).astype(np.float32)
    A = [mx.DeviceBuffer.from_numpy(a) for _ in range(20)]
    B = mx.DeviceBuffer.from_numpy(b)
    C = [mx.DeviceBuffer(a.nbytes) for _ in range(2)]
    S = mx.DeviceBuffer(4096 * 4)
    out, out_st, _, b1st, _, b2st = mx.broadcast_shapes([4096, 1024], [1024, 1], [1, 1024], [1024, 1])
    desc = mx.collapse_dims3(out, b1st, b2st, out_st)
    rdesc = mx.collapse_dims_reduce2([4096, 1024], [1], [1024, 1], 1)

    add = mx.prepare_bcast_binary(mx.OP_ADD, mx.FLOAT32, desc)
    rowsum = mx.prepare_reduce(mx.RED_SUM, mx.FLOAT32, 1, 1024, rdesc)
    fused = mx.prepare_bcast_binary_reduce_rows(mx.OP_ADD, mx.RED_SUM, mx.FLOAT32, desc, 1024)

    def graph(i=0):
        c = C[i % 2]
        add(c.ptr, A[i % 20].ptr, B.ptr)
        rowsum(S.ptr, c.ptr)

    def graph_fused(i=0):
        fused(C[i % 2].ptr, A[i % 20].ptr, B.ptr, S.ptr)

    graph_bytes, moved = 50_352_128, 33_574_912
    ms2 = _best(mx, graph, 40)
    ms = _best(mx, graph_fused, 40)
    gbs = moved / (ms * 1e-3) / 1e9
    return {"ms": round(ms, 5), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
            "hbm_bytes": moved, "graph_bytes": graph_bytes,
            "graph_GB/s": round(graph_bytes / (ms * 1e-3) / 1e9, 1),
            "unfused_ms": round(ms2, 5), "unfused_GB/s": round(graph_bytes / (ms2 * 1e-3) / 1e9, 1),
            "note": "the graph's add and row sum fused into one launch (C written, its rows reduced from "
                    "registers); GB/s / frac_hbm over the 33,574,912 bytes that launch moves, graph_GB/s over "
                    "the unfused graph's 50,352,128 algorithmic bytes, unfused_* the two launches",
            "_cpu_inputs": (a, b, desc, rdesc)}


def matmul_case(mx, dt, kind, rng):
    """(launch(i), flop or bytes, host operands, descriptor, K) of config 3's main product
    A[16,2048,2048] x B[2048,2048] (kind "main") or the skinny A[8,1,4096] x B[4096,4096]."""
    code = mx.FLOAT32 if dt == "f32" else mx.FLOAT16
    if kind == "main":
        a = _normal(rng, [16, 2048, 2048], 1 / np.sqrt(2048), dt)
        bt = _normal(rng, [2048, 2048], 1 / np.sqrt(2048), dt)
        desc = ([16, 2048, 2048], [2048 * 2048, 2048, 1], [0, 2048, 1], [2048 * 2048, 2048, 1])
        K, copies = 2048, 1
    else:
        a = _normal(rng, [8, 1, 4096], 1 / 64, dt)
        bt = _normal(rng, [4096, 4096], 1 / 64, dt)
        desc = ([8, 1, 4096], [4096, 4096, 1], [0, 4096, 1], [4096, 4096, 1])
        K, copies = 4096, (8 if dt == "f32" else 12)     # rotated copies of B: 256 MiB and more
    A = mx.DeviceBuffer.from_numpy(a)
    Bs = [mx.DeviceBuffer.from_numpy(bt) for _ in range(copies)]
    C = mx.DeviceBuffer(int(np.prod(desc[0])) * a.itemsize)
    wsb = mx.matmul_workspace_bytes(code, desc, K)
    W = mx.DeviceBuffer(wsb) if wsb else None
    mm = mx.prepare_batched_matmul(code, desc, K, workspace=W.ptr if W else 0, workspace_bytes=wsb)
    keep = (A, Bs, C, W)

    def launch(i=0):
        mm(C.ptr, A.ptr, Bs[i % copies].ptr)
    launch.keep = keep
    return launch, (a, bt, desc, K, code)


def matmul_graph_case(mx, dt, kind, rng):
    """launch(i) of config 3's product as the graph's A.dot(B) runs it from B stored [K, N], with
    no transposed copy of B: the tile kernel (main) or the streaming kernel (skinny, 8 rows of A)
    reads B N-major."""
    code = mx.FLOAT32 if dt == "f32" else mx.FLOAT16
    if kind == "main":
        a = _normal(rng, [16, 2048, 2048], 1 / np.sqrt(2048), dt)
        b = _normal(rng, [2048, 2048], 1 / np.sqrt(2048), dt)
        M, K, N, batch, copies = 2048, 2048, 2048, 16, 1
    else:
        a = _normal(rng, [8, 1, 4096], 1 / 64, dt)
        b = _normal(rng, [4096, 4096], 1 / 64, dt)
        M, K, N, batch, copies = 1, 4096, 4096, 8, (8 if dt == "f32" else 12)
    A = mx.DeviceBuffer.from_numpy(a)
    Bs = [mx.DeviceBuffer.from_numpy(b) for _ in range(copies)]
    C = mx.DeviceBuffer(batch * M * N * a.itemsize)
    desc = ([batch, M, N], [M * K, K, 1], [0, 1, N], [M * N, N, 1])          # Bt = B^T as a view
    wsb = mx.matmul_workspace_bytes(code, desc, K)
    W = mx.DeviceBuffer(wsb) if wsb else None
    mm = mx.prepare_batched_matmul(code, desc, K, workspace=W.ptr if W else 0, workspace_bytes=wsb)

    def launch(i=0):
        mm(C.ptr, A.ptr, Bs[i % copies].ptr)
    launch.keep = (A, Bs, C, W)
    return launch


def library_gemm_tflops(mx, dt, rng, reps=20):
    """Config 3's main product folded (C[32768, 2048] = A[32768, 2048] . B[2048, 2048]) through
    the vendor library on the same box -- rocBLAS's gemm_ex (f16 in, fp32 compute; fp32), called
    through ctypes on the same N(0,1)/sqrt(2048) data -- as a comparison point.  None when rocBLAS
    cannot be loaded or refuses the call."""
    import ctypes
    try:
        rb = ctypes.CDLL("librocblas.so")
    except OSError:
        try:
            rb = ctypes.CDLL("/opt/rocm/lib/librocblas.so")
        except OSError:
            return None
    M, N, K = 32768, 2048, 2048
    a = _normal(rng, [M, K], 1 / np.sqrt(2048), dt)
    bt = _normal(rng, [N, K], 1 / np.sqrt(2048), dt)
    A, B = mx.DeviceBuffer.from_numpy(a), mx.DeviceBuffer.from_numpy(bt)
    C = mx.DeviceBuffer(M * N * a.itemsize)
    h, stream = ctypes.c_void_p(), ctypes.c_void_p()
    if rb.rocblas_create_handle(ctypes.byref(h)) != 0:
        return None
    mx.check(mx.lib.mx_hip_stream_for_thread(ctypes.byref(stream)))    # the stream _timed's events see
    if rb.rocblas_set_stream(h, stream) != 0:
        rb.rocblas_destroy_handle(h)
        return None
    f16, f32 = 150, 151                                  # rocblas_datatype_f16_r / f32_r
    io = f16 if dt == "f16" else f32
    one, zero = ctypes.c_float(1.0), ctypes.c_float(0.0)
    # row-major C = A Bt^T is column-major C^T = Bt^T(op T of the [K x N] Bt) . A([K x M])
    args = (h, 112, 111, N, M, K, ctypes.byref(one), ctypes.c_void_p(B.ptr), io, K, ctypes.c_void_p(A.ptr), io, K,
            ctypes.byref(zero), ctypes.c_void_p(C.ptr), io, N, ctypes.c_void_p(C.ptr), io, N, f32, 0, 0, 0)

    def launch(i=0):
        st = rb.rocblas_gemm_ex(*args)
        if st != 0:
            raise RuntimeError(f"rocblas_gemm_ex status {st}")
    try:
        ms = _best(mx, launch, reps)
    except RuntimeError:
        return None
    finally:
        rb.rocblas_destroy_handle(h)
    return round(2.0 * M * N * K / (ms * 1e-3) / 1e12, 1)


def config_matmul(mx):
    """Config 3: A[16,2048,2048] x B[2048,2048] (B broadcast over the batch), f32 and f16 with
    fp32 accumulation; skinny A[8,1,4096] x B[4096,4096].  B^T is packed once (dot's copy) and
    the timed launches are the batched-matmul kernel alone."""
    rng = np.random.default_rng(1)
    res, cpu_in = {}, {}
    for dt in ("f32", "f16"):
        launch, host = matmul_case(mx, dt, "main", rng)
        ms = _best(mx, launch, 5 if dt == "f32" else 20)
        tf = 274_877_906_944 / (ms * 1e-3) / 1e12
        res[f"main_{dt}"] = {"ms": round(ms, 4), "TFLOP/s": round(tf, 1),
                             "frac_mfma": round(tf / MFMA_PEAK_TFLOPS[dt], 4),
                             "rocblas_TFLOP/s": library_gemm_tflops(mx, dt, rng),
                             "note": "rocblas_TFLOP/s: the vendor library on the same box, same folded product"}
        cpu_in[f"main_{dt}"] = host
        del launch
        launch, host = matmul_case(mx, dt, "skinny", rng)
        a, bt = host[0], host[1]
        ms = _best(mx, launch, 40)
        nbytes = (a.size + bt.size + 8 * 4096) * a.itemsize
        gbs = nbytes / (ms * 1e-3) / 1e9
        res[f"skinny_{dt}"] = {"ms": round(ms, 5), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
        cpu_in[f"skinny_{dt}"] = host
        del launch
        # the same products as the graph's A.dot(B) runs them from B stored [K, N]
        launch = matmul_graph_case(mx, dt, "main", rng)
        ms = _best(mx, launch, 5 if dt == "f32" else 20)
        tf = 274_877_906_944 / (ms * 1e-3) / 1e12
        res[f"main_{dt}_dot"] = {"ms": round(ms, 4), "TFLOP/s": round(tf, 1), "frac_mfma": round(tf / MFMA_PEAK_TFLOPS[dt], 4),
                                 "note": "B stored [K, N], read N-major by the tile kernel (no transposed copy)"}
        del launch
        launch = matmul_graph_case(mx, dt, "skinny", rng)
        ms = _best(mx, launch, 40)
        gbs = nbytes / (ms * 1e-3) / 1e9
        res[f"skinny_{dt}_dot"] = {"ms": round(ms, 5), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                                   "note": "B stored [K, N], read N-major by the streaming kernel (no transposed "
                                           "copy); GB/s over the product's A + B + C bytes"}
        del launch
    res["_cpu_inputs"] = cpu_in
    return res


def _cs(shape):
    st, acc = [0] * len(shape), 1
    for i in range(len(shape) - 1, -1, -1):
        st[i] = acc
        acc *= shape[i]
    return st


CONV_CASES = {"3x3": (32, 64, 56, 56, 128, 3, 1, 1), "1x1s2": (32, 256, 28, 28, 512, 1, 0, 2)}


def conv_geom(name, layout):
    """Channels-last geometry of config 4's case `name`: NCHW-stored tensors seen through the
    reference conv2d's transpose(0,2,3,1) views ("nchw"), or stored NHWC / OHWI ("nhwc")."""
    n, c, h, w, o, k, pad, stride = CONV_CASES[name]
    oh = (h + 2 * pad - k) // stride + 1
    ow = (w + 2 * pad - k) // stride + 1
    if layout == "nchw":
        st = _cs([n, c, h, w])
        in_st = [st[0], st[2], st[3], st[1]]
        kst = _cs([o, c, k, k])
        k_st = [kst[0], kst[2], kst[3], kst[1]]
    else:
        in_st, k_st = _cs([n, h, w, c]), _cs([o, k, k, c])
    return dict(in_shape=[n, h, w, c], k_shape=[o, k, k, c], out_shape=[n, oh, ow, o], in_strides=in_st,
                k_strides=k_st, out_strides=_cs([n, oh, ow, o]), pad=[pad, pad], stride=[stride, stride])


def conv_case(mx, dt, name, layout, rng):
    """(launch(i), flop, host operands) of one config-4 convolution (packing inside the call)."""
    code = mx.FLOAT32 if dt == "f32" else mx.FLOAT16
    n, c, h, w, o, k, pad, stride = CONV_CASES[name]
    geom = conv_geom(name, layout)
    x = _normal(rng, [n, c, h, w] if layout == "nchw" else [n, h, w, c], 1.0, dt)
    wt = _normal(rng, [o, c, k, k] if layout == "nchw" else [o, k, k, c], np.sqrt(2.0 / (c * k * k)), dt)
    X, W = mx.DeviceBuffer.from_numpy(x), mx.DeviceBuffer.from_numpy(wt)
    Y = mx.DeviceBuffer(int(np.prod(geom["out_shape"])) * x.itemsize)
    wsb = mx.conv_workspace_bytes(code, geom)
    WS = mx.DeviceBuffer(max(wsb, 256))
    conv = mx.prepare_conv_nd(code, geom, WS.ptr, wsb)

    def launch(i=0):
        conv(Y.ptr, X.ptr, W.ptr)
    launch.keep = (X, W, Y, WS)
    flop = 2.0 * np.prod(geom["out_shape"]) * c * k * k
    return launch, flop, (x, wt, geom, code)


def config_conv(mx):
    """Config 4: x [32,64,56,56] (NCHW) * w [128,64,3,3], stride 1, pad 1, fed as the reference's
    conv2d sees them (NHWC / OHWI transposed views: packing is part of the timed call) and
    natively channels-last; 1x1 stride 2: x [32,256,28,28] * w [512,256,1,1]."""
    rng = np.random.default_rng(2)
    res, cpu_in = {}, {}
    for dt in ("f32", "f16"):
        for name, layouts in (("3x3", ("nchw", "nhwc")), ("1x1s2", ("nchw", "nhwc"))):
            for layout in layouts:
                launch, flop, host = conv_case(mx, dt, name, layout, rng)
                ms = _best(mx, launch, 20)
                tf = flop / (ms * 1e-3) / 1e12
                res[f"{name}_{layout}_{dt}"] = {"ms": round(ms, 4), "TFLOP/s": round(tf, 1),
                                                "frac_mfma": round(tf / MFMA_PEAK_TFLOPS[dt], 4)}
                if layout == "nchw":
                    cpu_in[f"{name}_{dt}"] = host
                del launch
    res["_cpu_inputs"] = cpu_in
    return res


def graph_step(args):
    """The workload's compiled graph through the C++ graph API (a child process)."""
    import subprocess
    exe = os.path.join(ROOT, "matrix_amd", "_bin", "reductions_step")
    if not os.path.exists(exe):
        raise SystemExit("bench.py: matrix_amd/_bin/reductions_step is not built (python __graft_entry__.py build)")
    out = subprocess.run([exe, "--steps", str(args.steps), "--warmup", str(args.warmup)], capture_output=True,
                         text=True, timeout=300)
    if out.returncode != 0:
        raise SystemExit("bench.py: reductions_step failed: " + (out.stderr or out.stdout).strip()[-500:])
    return json.loads(out.stdout.strip().splitlines()[-1])


def config_mlp():
    """Config 5: the compiled-graph MLP training step through the C++ graph API (a child process)."""
    import subprocess
    exe = os.path.join(ROOT, "matrix_amd", "_bin", "mlp_step")
    if not os.path.exists(exe):
        return {"error": "matrix_amd/_bin/mlp_step not built"}
    out = subprocess.run([exe, "--steps", "30", "--warmup", "5"], capture_output=True, text=True, timeout=300)
    if out.returncode != 0:
        return {"error": (out.stderr or out.stdout).strip()[-300:]}
    r = json.loads(out.stdout.strip().splitlines()[-1])
    r["frac_mfma"] = round(r["tflops"] / MFMA_PEAK_TFLOPS["f32"], 4)
    return r


def cpu_info():
    """The host CPU model and its core counts, stated with every CPU baseline."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "nproc": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0))}


def _cpu_median(fn, reps, budget_s):
    """Median wall time of fn() over reps runs (fewer when the budget runs out, at least one)."""
    times, t_all = [], time.perf_counter()
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_all > budget_s:
            break
    return float(np.median(times)), len(times)


def run_cpu_baseline(mx_collapse):
    """The oracle (the reference's CPU loops restated) single-threaded on the host: the whole
    step's ops on the same X, repeated until about 10 s of CPU time; GB/s of algorithmic bytes."""
    from oracle import oracle as orc
    orc.load()
    x = make_input(0)
    inter = {}
    nbytes, reps, t0 = 0, 0, time.perf_counter()
    while True:
        for name, op, shape, axis, src, desc, rs, n, total, nb in mx_collapse:
            inp = x if src == "X" else inter[src]
            o = orc.reduce(op, orc.F32, rs, n, desc, total, inp, nthreads=1)
            inter[name] = o
            nbytes += nb
        reps += 1
        dt = time.perf_counter() - t0
        if dt > 10.0 or reps >= 40:
            break
    return {"value": round(nbytes / dt / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"the full step (all ops on X[256,65536] f32) x{reps}, {dt:.2f} s single-threaded",
            **cpu_info()}


def cpu_add_rowsum(orc, inputs):
    """Config 1 on the oracle, single-threaded: the add then the row sum (the reference's two
    CPU loops), median of 5; GB/s over the graph's 50,352,128 algorithmic bytes."""
    a, b, desc, rdesc = inputs

    def run():
        c = orc.bcast_binary(orc.ADD, orc.F32, desc, a.size, a.ravel(), b.ravel())
        orc.reduce(orc.RSUM, orc.F32, 1, 1024, rdesc, 4096, c, nthreads=1)
    sec, n = _cpu_median(run, 5, 20.0)
    return {"value": round(50_352_128 / sec / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"the whole graph (add + row sum of A[4096,1024]), median of {n}", **cpu_info()}


def cpu_matmul(orc, name, host):
    """Config 3 on the oracle, single-threaded, on a bounded sample: the main product's first 128
    (f32) or 32 (f16) rows of batch 0 (of 32768 rows), the skinny product whole.  f16 runs the reference's literal
    loop (half accumulator)."""
    a, bt, desc, K, code = host
    oc = orc.F32 if code == 0 else orc.F16
    if name.startswith("main"):
        rows = 128 if code == 0 else 32        # the literal half-accumulator loop is ~15x slower
        av = np.ascontiguousarray(a.reshape(-1, K)[:rows])
        d = ([rows, 2048], [K, 1], [K, 1], [2048, 1])
        flop = 2.0 * rows * 2048 * K
        sample = f"rows 0-{rows - 1} of batch 0 ({rows} x 2048 x {K}, {flop / 1e9:.2f} GFLOP)"
        total = rows * 2048
    else:
        av, d = a.reshape(-1), desc
        flop = 2.0 * 8 * 4096 * K
        sample = f"the whole product ({flop / 1e9:.2f} GFLOP)"
        total = 8 * 4096
    fn = (lambda: orc.batched_matmul(oc, d, K, av.reshape(-1), bt.reshape(-1), total, acc=orc.ACC_LITERAL,
                                     nthreads=1))
    sec, n = _cpu_median(fn, 3, 6.0)
    out = {"value": round(flop / sec / 1e12, 6), "unit": "TFLOP/s", "cores": 1, "kind": "port",
           "sample": f"{sample}, median of {n}", **cpu_info()}
    if not name.startswith("main"):
        nbytes = (a.size + bt.size + 8 * 4096) * a.itemsize
        out["GB/s"] = round(nbytes / sec / 1e9, 3)
    return out


def cpu_conv(orc, name, host):
    """Config 4 on the oracle, single-threaded, on a bounded sample: the first image(s) of the
    batch of 32, on the same NHWC / OHWI views of the NCHW tensors."""
    x, wt, geom, code = host
    oc = orc.F32 if code == 0 else orc.F16
    n_img = 1 if name.startswith("3x3") else (4 if code == 0 else 2)
    g = dict(geom)
    g["in_shape"] = [n_img] + geom["in_shape"][1:]
    g["out_shape"] = [n_img] + geom["out_shape"][1:]
    c = geom["in_shape"][-1]
    per_img = int(np.prod(geom["in_shape"][1:]))
    xs = np.ascontiguousarray(x.reshape(-1)[:n_img * per_img])       # NCHW: images are contiguous
    kk = geom["k_shape"][1] * geom["k_shape"][2]
    flop = 2.0 * np.prod(g["out_shape"]) * c * kk
    total = int(np.prod(g["out_shape"]))
    fn = (lambda: orc.conv(oc, g["in_shape"], g["k_shape"], g["out_shape"], g["in_strides"], g["k_strides"],
                           _cs(g["out_shape"]), g["pad"], g["stride"], [1, 1], [1, 1], 1, 0, xs, wt.reshape(-1),
                           total, acc=orc.ACC_LITERAL, nthreads=1))
    sec, n = _cpu_median(fn, 3, 6.0)
    return {"value": round(float(flop / sec / 1e12), 6), "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "sample": f"{n_img} of 32 images ({flop / 1e9:.2f} GFLOP), median of {n}", **cpu_info()}


def cpu_mlp(orc, batch=32):
    """Config 5 on the oracle, single-threaded: one training step of the same MLP at a batch of
    `batch` rows instead of 512 (the step's every op in the reference's CPU loops: the B^T copy
    dot makes before each product, the products, bias adds, the ReLU's Max and its four-node
    gradient, the loss and the bias gradients' column sums); steps/s at that batch and its
    TFLOP/s."""
    rng = np.random.default_rng(0)
    D = [1024, 4096, 4096, 10]
    B = batch
    F = orc.F32
    x = rng.standard_normal([B, D[0]], dtype=np.float32)
    t = rng.uniform(0, 1, [B, D[3]]).astype(np.float32)
    W = [(rng.standard_normal([D[l], D[l + 1]], dtype=np.float32) / np.sqrt(D[l])).astype(np.float32)
         for l in range(3)]
    bias = [np.zeros(D[l + 1], np.float32) for l in range(3)]
    zero = np.zeros(1, np.float32)
    one = np.ones(1, np.float32)

    def tr(m, r, c):          # contiguous copy of the transpose of m [r, c] (dot's B^T pack)
        return orc.copy_strided(F, F, [c, r], [r, 1], [1, c], np.empty(r * c, np.float32), m.reshape(-1))

    def mm(a, bt, M, N, K):   # a [M, K] . bt [N, K]^T
        return orc.batched_matmul(F, ([M, N], [K, 1], [K, 1], [N, 1]), K, a.reshape(-1), bt.reshape(-1), M * N,
                                  nthreads=1)

    def ew(op, a, b, n, b_scalar=False):
        return orc.bcast_binary(op, F, ([n], [1], [0 if b_scalar else 1], [1]), n, a.reshape(-1), b.reshape(-1))

    def add_rows(z, b, M, N):
        return orc.bcast_binary(orc.ADD, F, ([M, N], [N, 1], [0, 1], [N, 1]), M * N, z.reshape(-1), b)

    def col_sum(g, M, N):
        return orc.reduce(orc.RSUM, F, N, M, ([N], [1], [1]), N, g.reshape(-1), nthreads=1)

    def step():
        hs, zs, wts = [x], [], []
        for l in range(3):
            wt = tr(W[l], D[l], D[l + 1])
            wts.append(wt)
            z = add_rows(mm(hs[-1], wt, B, D[l + 1], D[l]), bias[l], B, D[l + 1])
            zs.append(z)
            hs.append(ew(orc.MAX, z, zero, B * D[l + 1], True) if l < 2 else z)
        n3 = B * D[3]
        d = ew(orc.SUB, hs[-1], t, n3)
        sq = ew(orc.MUL, d, d, n3)
        orc.reduce(orc.RSUM, F, 1, n3, ([1], [1], [n3]), 1, sq, nthreads=1)
        g = ew(orc.MUL, np.ones(n3, np.float32), d, n3)
        g = ew(orc.ADD, g, g, n3)                          # d(d*d) = g*d + g*d
        for l in (2, 1, 0):
            N, K = D[l + 1], D[l]
            col_sum(g, B, N)                               # bias gradient
            gt = tr(g, B, N)                               # g^T [N, B]
            ht = tr(hs[l], B, K)                           # h^T [K, B]
            mm(gt, ht, N, K, B)                            # (dW)^T = g^T . h
            if l > 0:
                ga = mm(g, tr(wts[l], N, K), B, K, N)      # g . W^T (dot packs W again)
                # the ReLU's vjp: mask = equal(0, max(z, 0)), g * (1 - mask) (primitives.cpp:2604-2608)
                m = ew(orc.MAX, zs[l - 1], zero, B * K, True)
                mask = orc.bcast_binary(orc.EQ, F, ([B * K], [0], [1], [1]), B * K, zero, m)
                keep = orc.bcast_binary(orc.SUB, F, ([B * K], [0], [1], [1]), B * K, one, mask)
                g = ew(orc.MUL, ga, keep, B * K)

    sec, n = _cpu_median(step, 3, 8.0)
    fwd = 2.0 * B * (D[0] * D[1] + D[1] * D[2] + D[2] * D[3])
    flop = fwd + 2.0 * fwd - 2.0 * B * D[0] * D[1]
    return {"value": round(1.0 / sec, 3), "unit": f"steps/s at batch {B}", "TFLOP/s": round(flop / sec / 1e12, 6),
            "cores": 1, "kind": "port",
            "sample": f"one training step at batch {B} of 512 ({flop / 1e9:.2f} GFLOP), median of {n}", **cpu_info()}


def measured_traffic(op_name):
    """HBM bytes per launch of op_name from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    measurement (scaled by the calibration copy), or None when that op was not measured."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f).get(op_name)
    except (OSError, ValueError):
        return None
    return rec["traffic_bytes"] if rec else None


MFMA_PROBES = {
    "matmul_main_f32": ("matmul", "f32", "main"), "matmul_main_f16": ("matmul", "f16", "main"),
    "conv_3x3_nhwc_f16": ("conv", "f16", "3x3", "nhwc"), "conv_3x3_nchw_f16": ("conv", "f16", "3x3", "nchw"),
    "conv_3x3_nhwc_f32": ("conv", "f32", "3x3", "nhwc"), "conv_1x1s2_nchw_f16": ("conv", "f16", "1x1s2", "nchw"),
}


def kernel_probe(op_name, reps=10):
    """For hardware-counter runs: only `op_name` -- an op or a group launch of the reductions
    workload (group_axis1, group_r4_axis3, ...) followed by a 256 MiB device copy (the calibration
    kernel of known bytes), or one of the matmul / convolution launches of MFMA_PROBES -- reps
    launches."""
    import matrix_amd as mx
    mx.init(0)
    if op_name in MFMA_PROBES:
        spec = MFMA_PROBES[op_name]
        rng = np.random.default_rng(1)
        if spec[0] == "matmul":
            launch, _ = matmul_case(mx, spec[1], spec[2], rng)
            flop = 274_877_906_944
        else:
            launch, flop, _ = conv_case(mx, spec[1], spec[2], spec[3], rng)
        for i in range(reps):
            launch(i)
        mx.sync()
        print(json.dumps({"probe": op_name, "launches": reps, "flop_per_launch": float(flop)}), flush=True)
        return
    x = make_input(0)
    copies = [mx.DeviceBuffer.from_numpy(x) for _ in range(N_COPIES)]
    prepared = [Prepared(mx, *o) for o in build_ops(mx)]
    groups = {g.name: g for g in (PreparedGroup(mx, [prepared[j] for j in idx]) for idx in make_groups(mx, prepared))}
    singles = {p.name: p for p in prepared}
    if op_name in groups:
        g = groups[op_name]
        if any(p.src != "X" for p in g.members):
            raise SystemExit(f"--kernel-probe: {op_name} reads intermediates; pick a group on X")
        for i in range(reps):
            g.launch([copies[(i * len(g.members) + k) % N_COPIES].ptr for k in range(len(g.members))])
        nbytes = g.bytes
    elif op_name in singles:
        p = singles[op_name]
        if p.src != "X":
            raise SystemExit(f"--kernel-probe: {op_name} reads an intermediate; pick an op on X")
        for i in range(reps):
            p.launch(mx, copies[i % N_COPIES].ptr)
        nbytes = p.bytes
    else:
        raise SystemExit(f"--kernel-probe: unknown op or group {op_name}")
    n = 64 << 20                                     # 256 MiB of float32
    src, dst = mx.DeviceBuffer(4 * n), mx.DeviceBuffer(4 * n)
    src.fill_bytes(0)
    for _ in range(reps):
        mx.launch_copy_strided(mx.FLOAT32, mx.FLOAT32, ([n], [1], [1]), dst.ptr, src.ptr)
    mx.sync()
    print(json.dumps({"probe": op_name, "launches": reps, "bytes_per_launch": nbytes,
                      "calibration_copy_bytes": 2 * 4 * n}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--kernel-probe", default=None, metavar="OP",
                    help="run only OP (an op or a group launch of the reductions workload, then a calibration "
                         "copy; or a matmul / convolution launch: " + ", ".join(MFMA_PROBES) + ") for counter runs")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="only the reductions workload")
    args = ap.parse_args()
    if args.kernel_probe:
        kernel_probe(args.kernel_probe)
        return 0
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "multi-GPU sharding is described in DESIGN.md, not run", file=sys.stderr)
        return 2
    r = run_gpu(args)
    g = graph_step(args)
    configs = {}
    if not args.no_configs:
        import matrix_amd as mx
        configs["add_rowsum_f32"] = config_add_rowsum(mx)
        configs["matmul"] = config_matmul(mx)
        configs["conv2d"] = config_conv(mx)
        configs["mlp_step_f32"] = config_mlp()
        cpu_in = {"add": configs["add_rowsum_f32"].pop("_cpu_inputs"), "matmul": configs["matmul"].pop("_cpu_inputs"),
                  "conv": configs["conv2d"].pop("_cpu_inputs")}
        if not args.no_cpu_baseline:
            # every config's CPU baseline: the oracle single-threaded on a bounded sample of that workload
            from oracle import oracle as orc
            orc.load()
            configs["add_rowsum_f32"]["cpu_baseline"] = cpu_add_rowsum(orc, cpu_in["add"])
            for k, host in cpu_in["matmul"].items():
                configs["matmul"][k]["cpu_baseline"] = cpu_matmul(orc, k, host)
            for k, host in cpu_in["conv"].items():
                configs["conv2d"][k.replace("_", "_nchw_")]["cpu_baseline"] = cpu_conv(orc, k, host)
            configs["mlp_step_f32"]["cpu_baseline"] = cpu_mlp(orc)
    cpu = None if args.no_cpu_baseline else run_cpu_baseline(r["cpu_ops"])
    if int(g["step_bytes"]) != r["step_bytes"]:
        raise SystemExit(f"bench.py: step bytes differ ({g['step_bytes']} vs {r['step_bytes']})")
    line = {
        "metric": "HBM GB/s (broadcast/reduce) + TFLOP/s (matmul/conv), % of MI355X roofline",
        "value": round(g["GB/s"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(g["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: X[256,65536] ~ N(0,1) float32, seed 0, 30% rows with duplicated maxima, "
                f"{N_COPIES} resident copies, one per reduction that reads X",
        "config": {"workload": "reductions X[256,65536] f32: Sum/Max/Min/ArgMax/ArgMin over axis 1 and 0, "
                               "reshape [64,4,4096,16] over axes 3 then 1",
                   "step_bytes": r["step_bytes"], "parallelism": "single GPU",
                   "executor": f"compiled graph, execute + wait per step, {g['streams']} streams"},
        "roofline": {"bound": "hbm", "achieved": round(r["achieved"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(r["achieved"] / HBM_PEAK_GBS, 4), "traffic": measured_traffic(r["dominant"]),
                     "traffic_source": "profiles/traffic.json: rocprofv3 FETCH_SIZE x 1.9996 + WRITE_SIZE for this "
                                       "kernel (counter passes run apart from the bench, not in this run)",
                     "kernel": r["dominant"], "members": r["dominant_members"],
                     "bytes_per_launch": r["dominant_bytes"], "avg_ms": round(r["dominant_ms"], 5)},
        "cpu_baseline": cpu,
        "launch_loop_one_stream": {"ms_per_step": round(r["ms_per_step"], 4), "GB/s": round(r["value"], 1),
                                   "note": "the step's group launches issued back to back from Python on one "
                                           "stream, no wait between steps"},
        "per_group_gbs": r["per_group_gbs"],
        "per_op_gbs": r["per_op_gbs"],
        "configs": configs,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
