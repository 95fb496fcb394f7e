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


def _normal(rng, shape, scale, dt):
    x = (rng.standard_normal(shape, dtype=np.float32) * np.float32(scale))
    return x.astype(np.float16) if dt == "f16" else x


def config_add_rowsum(mx):
    """Config 1: C = A[4096,1024] + B[1,1024] (broadcast), s = C.sum(1); 20 rotated copies of A
    (320 MiB, more than the Infinity Cache)."""
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

    nbytes = 50_352_128
    ms2 = _timed(mx, graph, 40)
    ms = _timed(mx, graph_fused, 40)
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"ms": round(ms, 5), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
            "bytes": nbytes, "hbm_bytes": 33_574_912, "hbm_GB/s": round(33_574_912 / (ms * 1e-3) / 1e9, 1),
            "unfused_ms": round(ms2, 5), "unfused_GB/s": round(nbytes / (ms2 * 1e-3) / 1e9, 1),
            "note": "the graph's add and row sum fused into one launch (C written, read back from registers); "
                    "GB/s counts the unfused graph's 50,352,128 algorithmic bytes, hbm_GB/s the 33,574,912 moved"}


def config_matmul(mx):
    """Config 3: A[16,2048,2048] x B[2048,2048] (B broadcast over the batch), f32 and f16 with
    fp32 accumulation; skinny A[8,1,4096] x B[4096,4096].  B^T is packed once (dot's copy) and
    the timed launches are the batched-matmul kernel alone."""
    rng = np.random.default_rng(1)
    res = {}
    for dt in ("f32", "f16"):
        code = mx.FLOAT32 if dt == "f32" else mx.FLOAT16
        a = _normal(rng, [16, 2048, 2048], 1 / np.sqrt(2048), dt)
        bt = _normal(rng, [2048, 2048], 1 / np.sqrt(2048), dt)
        A, Bt = mx.DeviceBuffer.from_numpy(a), mx.DeviceBuffer.from_numpy(bt)
        C = mx.DeviceBuffer(16 * 2048 * 2048 * a.itemsize)
        desc = ([16, 2048, 2048], [2048 * 2048, 2048, 1], [0, 2048, 1], [2048 * 2048, 2048, 1])
        mm = mx.prepare_batched_matmul(code, desc, 2048)
        ms = _timed(mx, lambda i=0: mm(C.ptr, A.ptr, Bt.ptr), 5 if dt == "f32" else 20)
        tf = 274_877_906_944 / (ms * 1e-3) / 1e12
        res[f"main_{dt}"] = {"ms": round(ms, 4), "TFLOP/s": round(tf, 1),
                             "frac_mfma": round(tf / MFMA_PEAK_TFLOPS[dt], 4)}
        del A, Bt, C
        # skinny: 8 copies of B rotated (256 MiB and more), bytes = A + B + C
        a = _normal(rng, [8, 1, 4096], 1 / 64, dt)
        bt = _normal(rng, [4096, 4096], 1 / 64, dt)
        A = mx.DeviceBuffer.from_numpy(a)
        Bs = [mx.DeviceBuffer.from_numpy(bt) for _ in range(8 if dt == "f32" else 12)]
        C = mx.DeviceBuffer(8 * 4096 * a.itemsize)
        desc = ([8, 1, 4096], [4096, 4096, 1], [0, 4096, 1], [4096, 4096, 1])
        mm = mx.prepare_batched_matmul(code, desc, 4096)
        ms = _timed(mx, lambda i=0: mm(C.ptr, A.ptr, Bs[i % len(Bs)].ptr), 40)
        nbytes = (a.size + bt.size + 8 * 4096) * a.itemsize
        gbs = nbytes / (ms * 1e-3) / 1e9
        res[f"skinny_{dt}"] = {"ms": round(ms, 5), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
        del A, Bs, C
    return res


def config_conv(mx):
    """Config 4: x [32,64,56,56] (NCHW) * w [128,64,3,3], stride 1, pad 1, fed as the reference's
    conv2d sees them (NHWC / OHWI transposed views: packing is part of the timed call) and
    natively channels-last; 1x1 stride 2: x [32,256,28,28] * w [512,256,1,1]."""
    rng = np.random.default_rng(2)

    def cs(shape):
        st, acc = [0] * len(shape), 1
        for i in range(len(shape) - 1, -1, -1):
            st[i] = acc
            acc *= shape[i]
        return st

    res = {}
    for dt in ("f32", "f16"):
        code = mx.FLOAT32 if dt == "f32" else mx.FLOAT16
        for name, (n, c, h, w, o, k, pad, stride), layouts in (
                ("3x3", (32, 64, 56, 56, 128, 3, 1, 1), ("nchw", "nhwc")),
                ("1x1s2", (32, 256, 28, 28, 512, 1, 0, 2), ("nchw",))):
            oh = (h + 2 * pad - k) // stride + 1
            ow = (w + 2 * pad - k) // stride + 1
            x = _normal(rng, [n, c, h, w], 1.0, dt)
            wt = _normal(rng, [o, c, k, k], np.sqrt(2.0 / (c * k * k)), dt)
            X, W = mx.DeviceBuffer.from_numpy(x), mx.DeviceBuffer.from_numpy(wt)
            Y = mx.DeviceBuffer(n * oh * ow * o * x.itemsize)
            for layout in layouts:
                if layout == "nchw":
                    st = cs([n, c, h, w])
                    in_st = [st[0], st[2], st[3], st[1]]
                    kst = cs([o, c, k, k])
                    k_st = [kst[0], kst[2], kst[3], kst[1]]
                else:
                    in_st, k_st = cs([n, h, w, c]), cs([o, k, k, c])
                geom = dict(in_shape=[n, h, w, c], k_shape=[o, k, k, c], out_shape=[n, oh, ow, o], in_strides=in_st,
                            k_strides=k_st, out_strides=cs([n, oh, ow, o]), pad=[pad, pad], stride=[stride, stride])
                wsb = mx.conv_workspace_bytes(code, geom)
                WS = mx.DeviceBuffer(max(wsb, 256))
                conv = mx.prepare_conv_nd(code, geom, WS.ptr, wsb)
                ms = _timed(mx, lambda i=0: conv(Y.ptr, X.ptr, W.ptr), 20)
                flop = 2.0 * n * oh * ow * o * c * k * k
                tf = flop / (ms * 1e-3) / 1e12
                res[f"{name}_{layout}_{dt}"] = {"ms": round(ms, 4), "TFLOP/s": round(tf, 1),
                                                "frac_mfma": round(tf / MFMA_PEAK_TFLOPS[dt], 4)}
                del WS
            del X, W, Y
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
            "sample": f"the full step (all ops on X[256,65536] f32) x{reps}, {dt:.2f} s single-threaded"}


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


def kernel_probe(op_name, reps=10):
    """For hardware-counter runs: only `op_name` of the reductions workload -- one op, or a group
    launch (group_axis1, group_r4_axis3, ...) -- reps launches on rotated copies, then a 256 MiB
    device copy (the calibration kernel of known bytes)."""
    import matrix_amd as mx
    mx.init(0)
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
                    help="run only OP (an op or a group launch) of the reductions workload and a calibration "
                         "copy (for counter runs)")
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
