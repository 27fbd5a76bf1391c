"""Build the gfx950 C-ABI library ``libecdecode.so`` from ``csrc/*.hip`` (in-tree).

Each translation unit is compiled with hipcc for gfx950 only, in parallel, then linked
into ``estudiocanciones_amd/_lib/libecdecode.so``.  No GPU is needed to build.

    python -m estudiocanciones_amd.build
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
OBJDIR = PKG / "_build"
LIBDIR = PKG / "_lib"
LIBNAME = "libecdecode.so"
ARCH = "gfx950"

# -packed-fp32-ops: hipcc must not emit packed fp32 VALU ops for this library.
HIPFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", f"-I{INCLUDE}", f"-I{CSRC}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the gfx950 library cannot be built")


# per-file additions: the layer-stack launch keeps constants and addresses inside its layer loop
# (hoisted out of it, they would hold registers across every layer)
FILE_FLAGS = {"layer_stack.hip": ["-mllvm", "-disable-machine-licm"]}


def _compile(src: Path) -> Path:
    obj = OBJDIR / (src.stem + ".o")
    cmd = [hipcc(), *HIPFLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{r.stderr}")
    return obj


def build(verbose: bool = True) -> Path:
    """Compile every csrc/*.hip for gfx950 and link the shared library. Returns its path."""
    OBJDIR.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = max(1, min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)), 16))
    with ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    out = LIBDIR / LIBNAME
    tmp = LIBDIR / (LIBNAME + ".tmp")
    # --no-undefined: a kernel whose host stub was not emitted fails here, not at load time
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,--no-undefined", "-o",
           str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out} from {len(srcs)} sources", file=sys.stderr)
    return out


if __name__ == "__main__":
    build()
