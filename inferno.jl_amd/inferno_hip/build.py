"""Compile the gfx950 HIP library in-tree.

    python -m inferno_hip.build        (from inferno.jl_amd/)

Produces inferno.jl_amd/lib/libinferno_hip.so from inferno.jl_amd/csrc/*.hip
with hipcc.  Flags:
  --offload-arch=gfx950                 MI355X code objects only
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                        no packed-fp32 VALU instructions
  -fno-gpu-flush-denormals-to-zero      IEEE denormals (bit-exact dequant)
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parents[1]          # inferno.jl_amd/
CSRC = PKG / "csrc"
LIBDIR = PKG / "lib"
LIB = LIBDIR / "libinferno_hip.so"
INCLUDE = PKG.parent / "include"

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-gpu-flush-denormals-to-zero",
    "-Wno-unused-command-line-argument",
]


CHECKS = PKG.parent / "tests" / "native"
CHECK_LIB = CHECKS / "_build" / "libsdig_check.so"


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


OBJDIR = PKG / "_build"


def _run(cmd, verbose: bool):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc failed ({r.returncode})")


def build(verbose: bool = False) -> Path:
    """Every source compiled to an object in parallel (no relocatable device
    code: each file's kernels are self-contained), then linked."""
    from concurrent.futures import ThreadPoolExecutor

    LIBDIR.mkdir(exist_ok=True)
    OBJDIR.mkdir(exist_ok=True)
    compile_flags = [f for f in FLAGS if f != "-shared"]
    objs = []
    cmds = []
    for src in sources():
        obj = OBJDIR / (src.stem + ".o")
        objs.append(obj)
        cmds.append([HIPCC, *compile_flags, "-c", f"-I{INCLUDE}", f"-I{CSRC}", "-o", str(obj), str(src)])
    workers = max(1, min(len(cmds), os.cpu_count() or 1, 8))
    with ThreadPoolExecutor(max_workers=workers) as ex:
        for f in [ex.submit(_run, c, verbose) for c in cmds]:
            f.result()
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, *FLAGS, "-o", str(tmp), *[str(o) for o in objs]], verbose)
    os.replace(tmp, LIB)
    return LIB


FLOORS_LIB = LIBDIR / "libinferno_floors.so"


def _hipcc(out: Path, srcs, verbose: bool) -> Path:
    out.parent.mkdir(parents=True, exist_ok=True)
    tmp = out.with_suffix(".so.tmp")
    cmd = [HIPCC, *FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-o", str(tmp), *[str(s) for s in srcs]]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc failed ({r.returncode})")
    os.replace(tmp, out)
    return out


def build_floors(verbose: bool = False) -> Path:
    """The benchmark's measurement kernels (empty launch, coalesced read):
    inferno.jl_amd/lib/libinferno_floors.so, loaded by bench.py only."""
    return _hipcc(FLOORS_LIB, [PKG / "floors" / "floors.hip"], verbose)


def build_checks(verbose: bool = False) -> Path:
    """Host-side checkers of the kernels' index arithmetic (tests/native): they
    include the headers the kernels form their indices with and run on the CPU."""
    return _hipcc(CHECK_LIB, [CHECKS / "sdig_check.hip", CHECKS / "prefill_check.hip"], verbose)


if __name__ == "__main__":
    print(build(verbose=True))
