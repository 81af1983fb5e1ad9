"""Build libsinkattn.so (gfx950) in-tree with hipcc.

    python -m sinkattn_amd.build          # or: python sinkattn_amd/build.py

Objects go to sinkattn_amd/_build/, the library to sinkattn_amd/libsinkattn.so, and the
measurement probe bench.py uses (csrc/probe/, not part of the library) to
sinkattn_amd/libsinkattn_probe.so.  All device code is compiled with packed-fp32
instructions disabled.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_PATH = PKG_DIR / "libsinkattn.so"
PROBE_PATH = PKG_DIR / "libsinkattn_probe.so"
PROBE_SOURCES = ["probe/valu_mix.hip"]
ARCH = os.environ.get("SINKATTN_ARCH", "gfx950")

SOURCES = [
    "block_sparse_fwd.hip",
    "pooling.hip",
    "pooling_generic.hip",
    "coverage_mask.hip",
    "compensation.hip",
    "qk_prep.hip",
    "noalloc.hip",
    "capi.cpp",
]

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-variable",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC)")


def _compile(src: str) -> Path:
    obj = BUILD_DIR / (src.replace("/", "_").rsplit(".", 1)[0] + ".o")
    cmd = [_hipcc(), *COMMON_FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
    if src.endswith(".cpp"):
        cmd[1:1] = ["-x", "hip"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    return obj


def _link(objs, path: Path) -> None:
    tmp = path.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, path)


def build(verbose: bool = True) -> Path:
    BUILD_DIR.mkdir(exist_ok=True)
    srcs = SOURCES + PROBE_SOURCES
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as pool:
        objs = list(pool.map(_compile, srcs))
    _link(objs[: len(SOURCES)], LIB_PATH)
    _link(objs[len(SOURCES):], PROBE_PATH)
    if verbose:
        print(f"built {LIB_PATH} and {PROBE_PATH.name}")
    return LIB_PATH


if __name__ == "__main__":
    build()
