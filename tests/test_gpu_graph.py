"""The C++ graph layer on the GPU (tests/cpp/graph_test.cpp, mode `gpu`): broadcast add then
row-sum, the fused broadcast + reduction across re-executions, reductions run as group launches,
reductions over views, batched dot, conv2d on NCHW views, a compiled MLP training step
(forward loss and every parameter gradient, executed three times with new inputs) and
value_and_grad, each against double-precision host loops of the same mathematics."""
import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

BIN = Path(__file__).resolve().parent / "cpp" / "_build" / "graph_test"


def test_graph_on_gpu():
    assert BIN.exists(), "build the C++ test drivers first (python matrix_amd/build.py --programs)"
    out = subprocess.run([str(BIN), "gpu"], capture_output=True, text=True, timeout=110)
    print(out.stdout)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "FAIL" not in out.stdout and out.stdout.count("PASS") == 11, out.stdout
