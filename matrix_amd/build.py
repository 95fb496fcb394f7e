"""Builds the gfx950 kernel library (and the oracle when asked) in-tree.

    python matrix_amd/build.py            # kernels -> matrix_amd/_lib/libmatrix_amd.so
    python matrix_amd/build.py --oracle   # also oracle/_build/liboracle.so

(Run by path: importing the package loads the library, which may be stale or absent.)

Objects are compiled in parallel with hipcc for gfx950 only; packed-fp32 instructions are
disabled for all device code.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIBDIR = PKG / "_lib"
LIB = LIBDIR / "libmatrix_amd.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}")
    # hipcc's host pass warns that it does not know the packed-fp32 feature; drop that line
    noise = [ln for ln in (proc.stdout + proc.stderr).splitlines()
             if ln.strip() and "packed-fp32-ops" not in ln and "is not a recognized feature" not in ln]
    if noise:
        sys.stderr.write("\n".join(noise) + "\n")


CXX = os.environ.get("MX_CXX", "/opt/rocm/llvm/bin/clang++")
HOST = PKG / "host"
CXX_FLAGS = ["-std=c++23", "-O2", "-fPIC", "-Wall", "-Wextra", "-Wno-unused-parameter",
             f"-I{ROOT / 'include'}"]


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def host_sources() -> list[Path]:
    return sorted(HOST.glob("*.cpp"))


def _stale(obj: Path, src: Path, deps: list[Path]) -> bool:
    if not obj.exists():
        return True
    t = obj.stat().st_mtime
    return any(p.stat().st_mtime > t for p in [src, *deps])


def build_kernels(jobs: int | None = None, incremental: bool = False) -> Path:
    """Compiles every source (incremental=True: only objects older than their source or any
    header of csrc/, host/ or include/) and links the library."""
    OBJ.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    srcs = sources()
    hsrcs = host_sources()
    headers = [*CSRC.glob("*.hpp"), *HOST.glob("*.hpp"), *(ROOT / "include").glob("*.h")]
    jobs_all = [([HIPCC, *HIP_FLAGS, "-c", str(s), "-o", str(OBJ / (s.stem + ".o"))], OBJ / (s.stem + ".o"), s)
                for s in srcs]
    jobs_all += [([CXX, *CXX_FLAGS, "-c", str(s), "-o", str(OBJ / ("host_" + s.stem + ".o"))],
                  OBJ / ("host_" + s.stem + ".o"), s) for s in hsrcs]
    cmds = [c for c, o, s in jobs_all if not incremental or _stale(o, s, headers)]
    objs = [o for _, o, _ in jobs_all]
    if not cmds and LIB.exists() and all(LIB.stat().st_mtime >= o.stat().st_mtime for o in objs):
        return LIB
    jobs = jobs or max(1, min(len(cmds), os.cpu_count() or 4, 8))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_run, c) for c in cmds]
        for f in futs:
            f.result()
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    return LIB


def build_oracle() -> Path:
    _run(["make", "-s", "-C", str(ROOT / "oracle")])
    return ROOT / "oracle" / "_build" / "liboracle.so"


PROGRAMS = PKG / "programs"
BINDIR = PKG / "_bin"
TESTS_CPP = ROOT / "tests" / "cpp"


def _link_program(src: Path, out: Path, rpath: str) -> None:
    out.parent.mkdir(exist_ok=True)
    _run([CXX, *CXX_FLAGS, str(src), "-o", str(out), f"-L{LIBDIR}", "-lmatrix_amd", f"-Wl,-rpath,{rpath}",
          "-Wl,-rpath,/opt/rocm/lib"])


def build_programs() -> list[Path]:
    """Workload drivers over the C++ graph API (matrix_amd/programs/*.cpp -> matrix_amd/_bin/)."""
    outs = []
    for src in sorted(PROGRAMS.glob("*.cpp")):
        out = BINDIR / src.stem
        _link_program(src, out, "$ORIGIN/../_lib")
        outs.append(out)
    return outs


def build_test_programs() -> list[Path]:
    """C++ test drivers (tests/cpp/*.cpp -> tests/cpp/_build/)."""
    outs = []
    for src in sorted(TESTS_CPP.glob("*.cpp")):
        out = TESTS_CPP / "_build" / src.stem
        _link_program(src, out, "$ORIGIN/../../../matrix_amd/_lib")
        outs.append(out)
    return outs


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--oracle", action="store_true", help="also build the CPU oracle")
    ap.add_argument("--programs", action="store_true", help="also build the workload and C++ test drivers")
    ap.add_argument("-j", type=int, default=None)
    ap.add_argument("--incremental", action="store_true", help="recompile only out-of-date objects")
    a = ap.parse_args(argv)
    print(build_kernels(a.j, incremental=a.incremental))
    if a.oracle:
        print(build_oracle())
    if a.programs:
        for p in build_programs() + build_test_programs():
            print(p)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
