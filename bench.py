#!/usr/bin/env python3
"""Throughput of the MI355X evaluation path on the reductions workload.

One step = every reduction of the workload on X[256, 65536] float32 (N(0,1), seed 0, 30% of
rows with duplicated extrema):
  Sum / Max / Min / ArgMax / ArgMin over axis 1 (long rows) and over axis 0 (strided columns),
  and on X.reshape(64, 4, 4096, 16): Sum / Max / Min over axis 3 then axis 1,
  ArgMax / ArgMin over axis 3 and over axis 1 separately.
`value` = algorithmic HBM bytes of the step (inputs read + outputs written) / step time, with
inputs resident in HBM and rotated over enough copies that the 256 MB Infinity Cache cannot
hold the working set.

Prints one JSON line.  `roofline` is the dominant kernel's bytes per launch over its average
duration (HIP events on the launch stream); `cpu_baseline` times the oracle (the reference's
CPU loops restated) single-threaded on a bounded sample on this host.
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
N_COPIES = 6          # 6 x 64 MiB inputs > 256 MB MALL


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
        if self.W:
            self.W.fill_bytes(0)      # arrival counters start at zero; launches leave them zero
        self.O = mx.DeviceBuffer(self.out_bytes)

    def launch(self, mx, in_ptr):
        mx.launch_reduce(self.op, mx.FLOAT32, self.rs, self.n, self.desc, self.O.ptr, in_ptr,
                         self.W.ptr if self.W else 0, self.ws)


def run_gpu(args):
    import matrix_amd as mx
    mx.init(0)
    x = make_input(0)
    copies = [mx.DeviceBuffer.from_numpy(x) for _ in range(N_COPIES)]
    prepared = [Prepared(mx, *o) for o in build_ops(mx)]
    by_name = {p.name: p for p in prepared}

    def step(i):
        # every op reading X gets the next resident copy, so no read of X can be served by the
        # Infinity Cache from an earlier op of the same step
        k = i * len(prepared)
        for j, p in enumerate(prepared):
            src = copies[(k + j) % N_COPIES].ptr if p.src == "X" else by_name[p.src].O.ptr
            p.launch(mx, src)

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

    # per-op durations (events bracket each op's launches on the same stream)
    per_op = {}
    reps = max(3, min(20, args.steps))
    for p in prepared:
        a, b = mx.Event(), mx.Event()
        a.record()
        for i in range(reps):
            src = copies[i % N_COPIES].ptr if p.src == "X" else by_name[p.src].O.ptr
            p.launch(mx, src)
        b.record()
        mx.sync()
        per_op[p.name] = a.elapsed_ms(b) / reps
    dom = max(prepared, key=lambda p: per_op[p.name])
    achieved = dom.bytes / (per_op[dom.name] * 1e-3) / 1e9
    return {
        "ms_per_step": ms_step, "wall_s": wall, "step_bytes": step_bytes,
        "value": step_bytes / (ms_step * 1e-3) / 1e9,
        "dominant": dom.name, "dominant_bytes": dom.bytes, "dominant_ms": per_op[dom.name],
        "achieved": achieved,
        "per_op_gbs": {k: round(by_name[k].bytes / (v * 1e-3) / 1e9, 1) for k, v in per_op.items()},
        "cpu_ops": [(p.name, p.op, p.shape, p.axis, p.src, p.desc, p.rs, p.n, p.total, p.bytes) for p in prepared],
    }


def run_cpu_baseline(mx_collapse):
    """The oracle (the reference's CPU loops restated) single-threaded on the host: the whole
    step's ops on the same X, repeated until about 5 s of CPU time; GB/s of algorithmic bytes."""
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
        if dt > 5.0 or reps >= 20:
            break
    return {"value": round(nbytes / dt / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"the full step (all ops on X[256,65536] f32) x{reps}, {dt:.2f} s single-threaded"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "multi-GPU sharding is described in DESIGN.md, not run", file=sys.stderr)
        return 2
    r = run_gpu(args)
    cpu = None if args.no_cpu_baseline else run_cpu_baseline(r["cpu_ops"])
    line = {
        "metric": "HBM GB/s (broadcast/reduce) + TFLOP/s (matmul/conv), % of MI355X roofline",
        "value": round(r["value"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: X[256,65536] ~ N(0,1) float32, seed 0, 30% rows with duplicated maxima, "
                f"{N_COPIES} resident copies rotated",
        "config": {"workload": "reductions X[256,65536] f32: Sum/Max/Min/ArgMax/ArgMin over axis 1 and 0, "
                               "reshape [64,4,4096,16] over axes 3 then 1",
                   "step_bytes": r["step_bytes"], "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(r["achieved"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(r["achieved"] / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": r["dominant"], "bytes_per_launch": r["dominant_bytes"],
                     "avg_ms": round(r["dominant_ms"], 5)},
        "cpu_baseline": cpu,
        "per_op_gbs": r["per_op_gbs"],
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
