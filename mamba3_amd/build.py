"""Build ``libmamba3_hip.so`` (gfx950) in-tree with hipcc.

Each ``csrc/*.hip`` translation unit is compiled in parallel, then linked into
``mamba3_amd/libmamba3_hip.so``. Run ``python -m mamba3_amd.build`` (or call
``build()``); ``__graft_entry__.build()`` calls it on every invocation.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIB_NAME = "libmamba3_hip.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
OBJ_DIR = os.path.join(ROOT, "_build")
SOURCES = ("abi.hip", "step.hip", "scan.hip", "chunk_state.hip", "linear.hip", "norm.hip",
           "noalloc.hip", "rscan.hip")
ARCH = os.environ.get("MAMBA3_OFFLOAD_ARCH", "gfx950")

# Packed FP32 ops are disabled in device code (a hardware-correctness precaution on this pool).
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
]


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the HIP library cannot be built")
    return path


def _compile(src: str, extra: list[str]) -> str:
    obj = os.path.join(OBJ_DIR, src.replace(".hip", ".o"))
    cmd = [_hipcc(), *COMMON_FLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr[-4000:]}")
    return obj


def build(verbose: bool = True, extra_flags: list[str] | None = None) -> str:
    """Compile every HIP source for ``ARCH`` and link the shared library; return its path."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    extra = list(extra_flags or [])
    with concurrent.futures.ThreadPoolExecutor(max_workers=len(SOURCES)) as pool:
        objs = list(pool.map(lambda s: _compile(s, extra), SOURCES))
    tmp = LIB_PATH + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr[-4000:]}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} for {ARCH}", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build()
