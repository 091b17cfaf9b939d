"""Builds libmlora.so, the HIP kernels of this package, for gfx950 with hipcc, in the source tree.

    python meepsquared_amd/_build.py [--jobs N]

(run by its path: `python -m meepsquared_amd._build` would import the package first, and the
package loads the library this script is about to rebuild).

Each `csrc/*.hip` file is compiled to an object in `csrc/_objs/` (in parallel) and the objects are
linked into `meepsquared_amd/_lib/libmlora.so`, which `meepsquared_amd._lib` loads.  Every call
compiles again: a stale library is never reused.
"""

import argparse
import concurrent.futures
import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OBJS = CSRC / "_objs"
LIBDIR = HERE / "_lib"
LIBRARY = LIBDIR / "libmlora.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# Packed fp32 arithmetic (v_pk_*_f32) stays off: some of its forms have given wrong results on these boxes.
FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wno-unused-command-line-argument"]


def _compile(src: Path) -> Path:
    obj = OBJS / (src.stem + ".o")
    cmd = [HIPCC, *FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{proc.stderr}")
    return obj


def build(jobs: int | None = None) -> Path:
    """Compiles every kernel source and links libmlora.so; returns its path."""
    OBJS.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    jobs = jobs or min(len(sources), max(1, (os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(jobs) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"linking libmlora.so failed:\n{proc.stderr}")
    # a symbol of this library left undefined (a kernel stub the host pass did not emit) would only
    # show when the library is loaded: refuse it here
    nm = subprocess.run(["nm", "-D", "--undefined-only", str(tmp)], capture_output=True, text=True)
    missing = [line.split()[-1] for line in nm.stdout.splitlines() if "mlora" in line]
    if nm.returncode == 0 and missing:
        raise RuntimeError(f"libmlora.so leaves its own symbols undefined: {missing[:5]}")
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    print(build(ap.parse_args().jobs))
    sys.exit(0)
