"""Build libdcengine.so (HIP, gfx950) in-tree.

    python -m directcompute_torch_amd.build        # or build() from Python

Each ``csrc/*.hip`` file is compiled to an object under ``_build/`` (in
parallel), then linked into ``directcompute_torch_amd/libdcengine.so``.  The
library is written atomically (temporary file + rename) so a concurrently
loading process never sees a half-written file.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import time

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(REPO, "_build")
LIB_NAME = "libdcengine.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
ARCH = os.environ.get("DCE_OFFLOAD_ARCH", "gfx950")

# Packed-FP32 instructions are disabled for every device pass (the host pass
# warns that it does not know the feature; that is expected).
HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: cannot build libdcengine.so")


def _compile(src: str, obj: str) -> str:
    cmd = [_hipcc(), *HIP_FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = True) -> str:
    """Compile and link the library; returns its path."""
    t0 = time.time()
    os.makedirs(BUILD_DIR, exist_ok=True)
    srcs = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))
    objs = []
    jobs = max(1, min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = []
        for s in srcs:
            obj = os.path.join(BUILD_DIR, s.replace(".hip", ".o"))
            objs.append(obj)
            futs.append(ex.submit(_compile, os.path.join(CSRC, s), obj))
        for f in futs:
            f.result()
    tmp = LIB_PATH + f".tmp{os.getpid()}"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"[dcengine] built {LIB_PATH} from {len(srcs)} sources in {time.time() - t0:.1f}s")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
