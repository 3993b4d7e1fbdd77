"""Build the gfx950 HIP library ``libalodlm_hip.so`` in-tree.

Each ``csrc/*.hip`` file is compiled with hipcc for gfx950 into an object in
``csrc/_build/`` and the objects are linked into ``alodlm_amd/libalodlm_hip.so``.
Run ``python -m alodlm_amd.build`` (or ``__graft_entry__.build()``).
"""

import concurrent.futures
import os
from pathlib import Path
import shutil
import subprocess
import sys

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE / "csrc"
BUILD = CSRC / "_build"
LIBRARY = PACKAGE / "libalodlm_hip.so"
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # Packed float32 instructions stay off (see the design notes).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result", "-Wno-unused-command-line-argument",
]


def hipcc():
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the ROCm toolchain is required to build the library")
    return path


def _compile(source):
    obj = BUILD / (source.stem + ".o")
    cmd = [hipcc(), *FLAGS, "-c", str(source), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{result.stderr[-8000:]}")
    return obj


def build(verbose=False):
    """Compile every csrc/*.hip for gfx950 and link libalodlm_hip.so."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    workers = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(workers) as pool:
        objects = list(pool.map(_compile, sources))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects),
           "-o", str(tmp)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"link failed:\n{result.stderr[-8000:]}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY} from {len(sources)} sources", file=sys.stderr)
    return LIBRARY


if __name__ == "__main__":
    build(verbose=True)
