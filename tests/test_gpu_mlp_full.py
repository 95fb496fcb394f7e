"""Config 5 at full size through the C++ graph API (matrix_amd/_bin/mlp_step): the 3-layer MLP
1024 -> 4096 -> 4096 -> 10, batch 512, float32, built and compiled once and executed repeatedly.
Every pre-activation (normwise <= 1e-5), the loss and every weight and bias gradient (normwise
<= 1e-4) of the last step are checked against a float64 recomputation of the same mathematics in
numpy (the forward pass, then the reference's vjp rules: primitives.cpp:5550-5567 for Dot,
:2604-2608 for the ReLU's Max with ties to the scalar, taking the ReLU masks from the GPU's
pre-activations, which may differ from float64's only within rounding of 0); and the executes must allocate no device memory (everything is allocated
by compile, .agents/MemoryManagement.md:24)."""
import json
import subprocess
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

EXE = Path(__file__).resolve().parent.parent / "matrix_amd" / "_bin" / "mlp_step"


def test_mlp_step_full_size(tmp_path):
    assert EXE.exists(), "build the workload drivers first (python matrix_amd/build.py --programs)"
    out = subprocess.run([str(EXE), "--steps", "3", "--warmup", "1", "--dump", str(tmp_path)], capture_output=True,
                         text=True, timeout=110)
    assert out.returncode == 0, out.stdout + out.stderr
    rec = json.loads(out.stdout.strip().splitlines()[-1])
    assert rec["allocs_during_execute"] == 0 and rec["frees_during_execute"] == 0, rec
    D = [1024, 4096, 4096, 10]
    B = 512

    def load(name, shape):
        return np.fromfile(tmp_path / f"{name}.bin", np.float32).reshape(shape).astype(np.float64)

    x, t = load("x", [B, D[0]]), load("t", [B, D[3]])
    W = [load(f"W{l}", [D[l], D[l + 1]]) for l in range(3)]
    b = [load(f"b{l}", [D[l + 1]]) for l in range(3)]
    zg = [load(f"z{l}", [B, D[l + 1]]) for l in range(3)]
    # forward in float64; each layer's pre-activation z against the GPU's, normwise
    hs, zs = [x], []
    for l in range(3):
        z = hs[-1] @ W[l] + b[l]
        zs.append(z)
        assert np.linalg.norm(zg[l] - z) <= 1e-5 * np.linalg.norm(z), f"z{l}"
        hs.append(np.maximum(z, 0.0) if l < 2 else z)
    d = hs[-1] - t
    loss = float((d * d).sum())
    got_loss = float(np.fromfile(tmp_path / "loss.bin", np.float32)[0])
    assert abs(got_loss - loss) <= 1e-4 * abs(loss), (got_loss, loss)
    # backward: g = dloss/dy = 2 d; the ReLU passes g where z > 0 (a tie z == 0 goes to the
    # scalar).  Its mask is the GPU's own (z computed in fp32): a pre-activation within fp32
    # rounding of 0 may fall on either side, and one flipped entry moves a whole column of the
    # next weight gradient by ~7e-4 normwise.  Flips are allowed only where |z| < 1e-4.
    masks = []
    for l in range(2):
        m_gpu, m_64 = zg[l] > 0, zs[l] > 0
        flips = m_gpu != m_64
        assert np.all(np.abs(zs[l][flips]) < 1e-4), f"ReLU mask of layer {l} differs away from 0"
        masks.append(m_gpu)
    hs_g = [x] + [np.maximum(zg[l], 0.0) for l in range(2)]
    g = 2.0 * d
    gW, gb = [None] * 3, [None] * 3
    for l in (2, 1, 0):
        gW[l] = hs_g[l].T @ g
        gb[l] = g.sum(0)
        if l > 0:
            g = (g @ W[l].T) * masks[l - 1]
    for l in range(3):
        gw = np.fromfile(tmp_path / f"gW{l}.bin", np.float32).reshape(D[l], D[l + 1])
        gbv = np.fromfile(tmp_path / f"gb{l}.bin", np.float32)
        assert np.linalg.norm(gw - gW[l]) <= 1e-4 * np.linalg.norm(gW[l]), f"dW{l}"
        assert np.linalg.norm(gbv - gb[l]) <= 1e-4 * np.linalg.norm(gb[l]), f"db{l}"
