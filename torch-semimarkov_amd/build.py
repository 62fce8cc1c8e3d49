"""Build libtsm_hip.so (HIP kernels + C ABI) in-tree for gfx950.

    python torch-semimarkov_amd/build.py [--jobs N] [--arch gfx950]

Each csrc/*.hip file is compiled separately (in parallel) and linked into
torch_semimarkov_amd/_lib/libtsm_hip.so.  The library depends only on the HIP
runtime; its C ABI is declared in include/tsm_hip.h.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "torch_semimarkov_amd", "_lib")
LIB = os.path.join(OUT_DIR, "libtsm_hip.so")
BUILD_DIR = os.path.join(HERE, "_build")

# -packed-fp32-ops off: packed FP32 forms are kept out of the generated code.
HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"),
]


def hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libtsm_hip.so)")


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(
        ln for ln in (r.stderr or "").splitlines() if "packed-fp32-ops" not in ln
    )
    if r.returncode != 0:
        raise RuntimeError(f"command failed: {' '.join(cmd)}\n{err}")
    return err


def build(arch: str = "gfx950", jobs: int = 4, verbose: bool = False) -> str:
    cc = hipcc()
    os.makedirs(BUILD_DIR, exist_ok=True)
    os.makedirs(OUT_DIR, exist_ok=True)
    # largest translation units first so the parallel build ends together
    srcs = sorted((f for f in os.listdir(CSRC) if f.endswith(".hip")),
                  key=lambda f: (-os.path.getsize(os.path.join(CSRC, f)), f))
    objs = []
    cmds = []
    for f in srcs:
        obj = os.path.join(BUILD_DIR, f.replace(".hip", ".o"))
        objs.append(obj)
        cmds.append([cc, f"--offload-arch={arch}", *HIP_FLAGS, "-c", os.path.join(CSRC, f), "-o", obj])
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        for msg in ex.map(_run, cmds):
            if verbose and msg.strip():
                print(msg, file=sys.stderr)
    tmp = LIB + ".tmp"
    _run([cc, f"--offload-arch={arch}", "-shared", "-fPIC", *objs, "-o", tmp])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--arch", default="gfx950")
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 4))
    ap.add_argument("-v", "--verbose", action="store_true")
    a = ap.parse_args()
    print(build(a.arch, a.jobs, a.verbose))
