"""The reference's graph API spellings and forward-mode autodiff (tests/cpp/api_test.cpp):
compile_metal / execute_metal / eval_metal, at<T>(), the variadic matrix::eval and detach,
leaf_scalar / mark_changed / invalidate_pass, make_leaf, jit_graph_gpu / grad_graph_gpu /
multi_jit_graph_gpu, value_and_grad / grad on one matrix, Primitive::get_inputs and jvp
(Matrix.mm:1076-1175, 1413-1470, 2677-2691, 8436-8469; matrix.h:1722-1764; primitives.cpp:110-117).
The CPU mode checks graph building only; the GPU mode evaluates against float64 host loops,
including the jvp of a 3-layer MLP against central finite differences in float64."""
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
BIN = ROOT / "tests" / "cpp" / "_build" / "api_test"


def ensure_built():
    if not BIN.exists():
        import importlib.util
        spec = importlib.util.spec_from_file_location("_mx_build", ROOT / "matrix_amd" / "build.py")
        b = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(b)
        b.build_test_programs()
    return BIN


def test_api_cpu():
    out = subprocess.run([str(ensure_built()), "cpu"], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "FAIL" not in out.stdout and out.stdout.count("PASS") == 3, out.stdout


@pytest.mark.gpu
def test_api_gpu():
    out = subprocess.run([str(BIN), "gpu"], capture_output=True, text=True, timeout=110)
    print(out.stdout)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "FAIL" not in out.stdout and out.stdout.count("PASS") == 4, out.stdout
