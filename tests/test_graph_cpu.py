"""The C++ graph layer without a device: shape inference, views, errors and the structure of
the gradient graph (tests/cpp/graph_test.cpp, mode `cpu`)."""
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
BIN = ROOT / "tests" / "cpp" / "_build" / "graph_test"


def ensure_built():
    if not BIN.exists():
        import importlib.util
        spec = importlib.util.spec_from_file_location("_mx_build", ROOT / "matrix_amd" / "build.py")
        b = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(b)
        b.build_test_programs()
    return BIN


def test_graph_building_cpu():
    out = subprocess.run([str(ensure_built()), "cpu"], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "FAIL" not in out.stdout and out.stdout.count("PASS") == 5, out.stdout
