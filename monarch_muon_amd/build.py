"""Build ``libmmuon.so`` (gfx950) in-tree with hipcc.

``python -m monarch_muon_amd.build`` compiles every ``csrc/*.hip`` to an object
in parallel and links the shared library next to this file.  hipcc
cross-compiles for gfx950 without a GPU.  ``build_probe()`` builds the
bench-only HBM streaming probe (``bench_probe.hip`` beside ``bench.py``) into a
library of its own, apart from the optimizer's.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
LIB = HERE / "libmmuon.so"
ARCH = "gfx950"

CFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # every rounding the reference performs is explicit; no silent FMA contraction
    "-ffp-contract=off",
    # packed fp32 VALU ops are disabled for every kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build libmmuon.so")
    return exe


def _compile(src: Path, obj: Path) -> None:
    cmd = [_hipcc(), *CFLAGS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        msg = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in l)
        raise RuntimeError(f"hipcc failed on {src.name}:\n{msg}")


def build(verbose: bool = True) -> Path:
    srcs = sorted(CSRC.glob("*.hip"))
    objdir = HERE / "_build"
    objdir.mkdir(exist_ok=True)
    objs = [objdir / (s.stem + ".o") for s in srcs]
    jobs = max(1, min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))
    with cf.ThreadPoolExecutor(jobs) as ex:
        list(ex.map(_compile, srcs, objs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources", file=sys.stderr)
    return LIB


def build_probe(verbose: bool = True) -> Path:
    """``bench_probe.so`` from ``bench_probe.hip`` at the repository root (used
    only by ``bench.py --hbm-ceiling`` / ``--data-energy``)."""
    root = HERE.parent
    src, out = root / "bench_probe.hip", root / "bench_probe.so"
    tmp = out.with_suffix(".so.tmp")
    cmd = [_hipcc(), *CFLAGS, "-shared", f"-I{root}", str(src), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        msg = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in l)
        raise RuntimeError(f"hipcc failed on {src.name}:\n{msg}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}", file=sys.stderr)
    return out


if __name__ == "__main__":
    build()
