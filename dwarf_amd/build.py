"""Build libdsqg_hip.so (the C-ABI HIP library) in-tree for gfx950.

Each ``csrc/*.hip`` file is compiled to an object by its own ``hipcc`` process (in parallel),
then the objects are linked into ``dwarf_amd/libdsqg_hip.so``.  Usage:

    python -m dwarf_amd.build            # build (always recompiles)
    python -m dwarf_amd.build --jobs 4
"""

from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
import time
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
INCLUDE = PKG_DIR.parent / "include"
LIB_NAME = "libdsqg_hip.so"
LIB_PATH = PKG_DIR / LIB_NAME
OBJ_DIR = PKG_DIR / "_build"

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Packed-FP32 VALU forms are kept out of the generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Kernel arguments ahead of any by-value parameter block (the decode step's position and row
    # pointers) arrive preloaded in scalar registers: no argument round trip before the first load.
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wno-unused-command-line-argument",
]
# Set DSQG_RESOURCE_USAGE=1 to print per-kernel VGPR / LDS / spill figures while compiling.
if os.environ.get("DSQG_RESOURCE_USAGE"):
    HIPCC_FLAGS += ["-Rpass-analysis=kernel-resource-usage"]


def hipcc_path() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (expected /opt/rocm/bin/hipcc)")


def _compile(src: Path, hipcc: str) -> tuple[Path, float, str]:
    obj = OBJ_DIR / (src.stem + ".o")
    t0 = time.time()
    cmd = [hipcc, *HIPCC_FLAGS, f"-I{INCLUDE}", "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    log = "\n".join(l for l in (res.stdout + res.stderr).splitlines()
                    if "packed-fp32-ops" not in l and l.strip())
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{log}")
    return obj, time.time() - t0, log


def build(jobs: int | None = None, verbose: bool = True) -> Path:
    """Compile every csrc/*.hip for gfx950 and link libdsqg_hip.so; returns its path."""
    hipcc = hipcc_path()
    OBJ_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(sources), max(1, (os.cpu_count() or 2)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        results = list(ex.map(lambda s: _compile(s, hipcc), sources))
    for obj, dt, log in results:
        if verbose:
            print(f"[dwarf_amd.build] {obj.name}: {dt:.1f}s", flush=True)
            if log:
                print(log, flush=True)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *[str(o) for o, _, _ in results]]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"[dwarf_amd.build] linked {LIB_PATH}", flush=True)
    return LIB_PATH


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=None)
    args = ap.parse_args(argv)
    build(args.jobs)
    return 0


if __name__ == "__main__":
    sys.exit(main())
