"""Build libeth_amd.so (every HIP kernel + the C-ABI) for gfx950 with hipcc.

Usage: python -m eth_amd.build  (or eth_amd.build.build()).  Objects go to
eth_amd/_build/, the shared library to eth_amd/libeth_amd.so, in-tree so it
travels with the source snapshot.
"""

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
INCLUDE = PKG.parent / "include"
OUT = PKG / "libeth_amd.so"
BUILD_DIR = PKG / "_build"

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wno-unused-result",
    # keep the compiler from emitting packed fp32 VALU ops
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc_path():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; the eth_amd HIP library cannot be built")


def sources():
    return sorted(CSRC.glob("*.hip"))


def _compile(src, obj, hipcc):
    cmd = [hipcc, *HIPCC_FLAGS, f"-I{INCLUDE}", "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr}")
    return obj


def build(verbose=True, jobs=None):
    hipcc = hipcc_path()
    BUILD_DIR.mkdir(exist_ok=True)
    srcs = sources()
    objs = [BUILD_DIR / (s.stem + ".o") for s in srcs]
    jobs = jobs or min(8, len(srcs), os.cpu_count() or 1)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        list(pool.map(lambda so: _compile(so[0], so[1], hipcc), zip(srcs, objs)))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT} from {len(srcs)} sources", flush=True)
    return OUT


if __name__ == "__main__":
    build()
    sys.exit(0)
