"""GPU: the weight-resident halo convolution against the implicit-GEMM tile kernel, bit for bit.

Both kernels accumulate each output's K = (kernel position, channel) terms in the same order (one
chain of MFMAs over K blocks of 16, fp32 accumulation, one rounding on store), so for the same
16-bit same convolution they must give the same bits; each is also checked against the oracle in
test_gpu_conv.py.  The library reads MATRIX_AMD_CONV_HALO once per process, so the tile kernel's
results come from a child process started with it set to 0.
"""
import json
import os
import subprocess
import sys
import tempfile

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CASES = [
    # (N, H, W, C, O, kh, kw, pad, dil, dtype)
    (4, 56, 56, 64, 128, 3, 3, 1, 1, "FLOAT16"),    # config 4's 3x3 case at batch 4: 196 tiles
    (3, 20, 33, 40, 200, 3, 3, 2, 2, "BFLOAT16"),   # dilation, padded channels, a 72-channel group
    (2, 31, 17, 64, 128, 1, 3, 1, 1, "FLOAT16"),    # a 1 x 3 kernel, a 16-row tail tile
    (2, 20, 22, 128, 192, 1, 3, 1, 1, "FLOAT16"),   # 128 channels: 2 K pairs per pixel, 6 in all
    (3, 9, 13, 130, 128, 3, 1, 1, 1, "BFLOAT16"),   # 130 channels padded to 192: 3 K pairs per pixel, 9 in all
]

# run in this process and, with the tile kernel forced, in a child process
RUNNER = r'''
import numpy as np


def _strides(shape):
    st, acc = [0] * len(shape), 1
    for i in range(len(shape) - 1, -1, -1):
        st[i] = acc
        acc *= shape[i]
    return st


def _store(x, dt):
    if dt == "FLOAT16":
        return x.astype(np.float16).view(np.uint16)
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)     # round to nearest even


def run_case(mx, case):
    n, h, w, c, o, kh, kw, pad, dil, dt = case
    rng = np.random.default_rng(n * 1009 + h * 31 + w + c + o)
    x = _store(rng.standard_normal([n, h, w, c]).astype(np.float32), dt)
    k = _store((rng.standard_normal([o, kh, kw, c]) * np.sqrt(2.0 / (c * kh * kw))).astype(np.float32), dt)
    out_shape = [n, h, w, o]
    geom = dict(in_shape=[n, h, w, c], k_shape=[o, kh, kw, c], out_shape=out_shape,
                in_strides=_strides([n, h, w, c]), k_strides=_strides([o, kh, kw, c]),
                out_strides=_strides(out_shape), pad=[pad if kh > 1 else 0, pad if kw > 1 else 0],
                stride=[1, 1], dil=[dil, dil])
    code = getattr(mx, dt)
    X, K = mx.DeviceBuffer.from_numpy(x.reshape(-1)), mx.DeviceBuffer.from_numpy(k.reshape(-1))
    total = int(np.prod(out_shape))
    Y = mx.DeviceBuffer(total * 2)
    Y.fill_bytes(0xFF)
    wsb = mx.conv_workspace_bytes(code, geom)
    WS = mx.DeviceBuffer(max(wsb, 256))
    mx.launch_conv_nd(code, geom, Y.ptr, X.ptr, K.ptr, WS.ptr, wsb)
    mx.sync()
    return Y.download(np.uint16, total)
'''

CHILD = r'''
import json, sys
import numpy as np
sys.path.insert(0, sys.argv[1])
import matrix_amd as mx
ns = {}
exec(sys.argv[2], ns)
mx.init(0)
cases = json.loads(sys.argv[3])
np.savez(sys.argv[4], *[ns["run_case"](mx, tuple(c)) for c in cases])
print("child done", flush=True)
'''


def test_halo_kernel_equals_tile_kernel(mx):
    ns = {}
    exec(RUNNER, ns)
    halo = [ns["run_case"](mx, case) for case in CASES]
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "tile.npz")
        env = dict(os.environ, MATRIX_AMD_CONV_HALO="0")
        proc = subprocess.run([sys.executable, "-c", CHILD, ROOT, RUNNER, json.dumps(CASES), path], env=env,
                              capture_output=True, text=True, timeout=110)
        assert proc.returncode == 0, proc.stdout + proc.stderr
        with np.load(path) as z:
            tile = [z[f"arr_{i}"] for i in range(len(CASES))]
    for case, a, b in zip(CASES, halo, tile):
        assert not np.all(a == 0xFFFF), case              # the output was written
        assert np.array_equal(a, b), (case, int(np.count_nonzero(a != b)))
