"""Result dtypes of the graph layer's binary ops (tests/cpp/dtype_test.cpp): promote_types against
the reference's 13 x 13 type_rules table (matrix.h:166-180), scalar_operand_type's rules
(matrix.h:1815-1840), and the cast nodes operator+ - * / and max / min / equal insert
(Matrix.mm:8312-8315) -- on the CPU; and mixed-dtype graphs evaluated on the GPU, each result
bit-exact against the oracle run in the promoted dtype on the same operands."""
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
BIN = ROOT / "tests" / "cpp" / "_build" / "dtype_test"

NP = {0: np.float32, 1: np.uint16, 2: np.uint8, 3: np.int32, 4: np.int16, 5: np.uint32, 6: np.uint16,
      7: np.uint8, 8: np.int8, 10: np.uint16, 11: np.int64, 12: np.uint64}


def ensure_built():
    if not BIN.exists():
        import importlib.util
        spec = importlib.util.spec_from_file_location("_mx_build", ROOT / "matrix_amd" / "build.py")
        b = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(b)
        b.build_test_programs()
    return BIN


def test_promotion_rules_cpu():
    out = subprocess.run([str(ensure_built()), "cpu"], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "FAIL" not in out.stdout and out.stdout.count("PASS") == 3, out.stdout


def _shape(s):
    return [int(x) for x in s.split(",")] if s else []


@pytest.mark.gpu
def test_mixed_dtype_graphs_gpu(tmp_path, orc):
    import matrix_amd as mx
    out = subprocess.run([str(BIN), "gpu", str(tmp_path)], capture_output=True, text=True, timeout=110)
    print(out.stdout)
    assert out.returncode == 0, out.stdout + out.stderr
    lines = (tmp_path / "manifest.txt").read_text().split()
    assert len(lines) == 11
    for line in lines:
        name, op, adt, ash, bdt, bsh, rdt, rsh = line.split("|")
        op, adt, bdt, rdt = int(op), int(adt), int(bdt), int(rdt)
        ash, bsh, rsh = _shape(ash), _shape(bsh), _shape(rsh)
        a = np.fromfile(tmp_path / f"{name}_a.bin", NP[adt])
        b = np.fromfile(tmp_path / f"{name}_b.bin", NP[bdt])
        got = np.fromfile(tmp_path / f"{name}_r.bin", NP[rdt])

        def cast(x, src, shape):
            if src == rdt:
                return x
            n = int(np.prod(shape)) if shape else 1
            st = mx.contiguous_strides(shape) if shape else [1]
            dst = np.zeros(n, NP[rdt])
            return orc.copy_strided(rdt, src, shape or [1], st, st, dst, x)

        ac, bc = cast(a, adt, ash), cast(b, bdt, bsh)
        o, o_st, b1, b1st, b2, b2st = mx.broadcast_shapes(ash, mx.contiguous_strides(ash) if ash else [],
                                                          bsh, mx.contiguous_strides(bsh) if bsh else [])
        assert list(o) == rsh, name
        desc = mx.collapse_dims3(o, b1st, b2st, o_st)
        ref = orc.bcast_binary(op, rdt, desc, int(np.prod(rsh)), ac, bc)
        assert np.array_equal(got.view(np.uint8), ref.astype(NP[rdt]).view(np.uint8)), name
