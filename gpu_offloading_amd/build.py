"""Build libkvc.so (all HIP sources of csrc/) for gfx950 with hipcc.

One shared library, compiled in-tree so that it travels with the repository:
    gpu_offloading_amd/lib/libkvc.so
Flags: -O3, C++17, gfx950 only, packed-FP32 instruction selection disabled
(``-Xclang -target-feature -Xclang -packed-fp32-ops``; hipcc's host pass
warns that it does not know the feature, which is harmless).
"""
from __future__ import annotations

import glob
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
INCLUDE = os.path.join(REPO_DIR, "include")
LIB_DIR = os.path.join(PKG_DIR, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libkvc.so")
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libkvc.so)")


STAMP_PATH = LIB_PATH + ".srchash"


def sources() -> list[str]:
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")))


def source_hash() -> str:
    """SHA-256 of everything libkvc.so is built from (sources, headers,
    flags): a library whose stamp differs was built from other sources."""
    import hashlib

    h = hashlib.sha256()
    files = sources() + sorted(glob.glob(os.path.join(CSRC, "*.h"))) + \
        [os.path.join(INCLUDE, "kvc.h")]
    for path in files:
        h.update(os.path.basename(path).encode())
        with open(path, "rb") as f:
            h.update(f.read())
    h.update(" ".join(HIP_FLAGS).encode())
    return h.hexdigest()


def _run(cmd: list[str]) -> tuple[int, list[str]]:
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature"
    return res.returncode, [ln for ln in (res.stdout + res.stderr).splitlines()
                            if noise not in ln]


def build_library(verbose: bool = False, jobs: int | None = None) -> str:
    """Compile every csrc/*.hip into libkvc.so (always recompiles): one hipcc
    process per source file, in parallel, then one link."""
    from concurrent.futures import ThreadPoolExecutor

    os.makedirs(LIB_DIR, exist_ok=True)
    obj_dir = os.path.join(LIB_DIR, "obj")
    os.makedirs(obj_dir, exist_ok=True)
    srcs = sources()
    objs = [os.path.join(obj_dir, os.path.basename(s)[:-4] + ".o") for s in srcs]
    cmds = [[hipcc(), *HIP_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", s, "-o", o]
            for s, o in zip(srcs, objs)]
    jobs = jobs or min(len(cmds), max(1, min(os.cpu_count() or 1, 16)))
    if verbose:
        for c in cmds:
            print(" ".join(c), flush=True)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        results = list(ex.map(_run, cmds))
    failed = [(s, m) for s, (rc, m) in zip(srcs, results) if rc != 0]
    if failed:
        raise RuntimeError("hipcc failed:\n" + "\n".join(
            f"{s}:\n" + "\n".join(m) for s, m in failed))
    msgs = [ln for _, m in results for ln in m]
    tmp = LIB_PATH + ".tmp"
    link = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    if verbose:
        print(" ".join(link), flush=True)
    rc, lm = _run(link)
    if rc != 0:
        raise RuntimeError("hipcc link failed:\n" + "\n".join(lm))
    msgs += lm
    if verbose and msgs:
        print("\n".join(msgs), file=sys.stderr)
    os.replace(tmp, LIB_PATH)
    with open(STAMP_PATH, "w") as f:
        f.write(source_hash() + "\n")
    return LIB_PATH


if __name__ == "__main__":
    print(build_library(verbose=True))
