"""Builds libwsl.so (the HIP kernels + C ABI) for gfx950 with hipcc.

Each ``csrc/*.hip`` is compiled to an object in ``_build/`` and the objects are linked
into ``weightshared_torchtitan_amd/libwsl.so`` in-tree, so the library travels with the
source tree. Run ``python -m weightshared_torchtitan_amd.build``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_PATH = os.path.join(PKG_DIR, "libwsl.so")
REPO_ROOT = os.path.dirname(PKG_DIR)
INCLUDE_DIR = os.path.join(REPO_ROOT, "include")

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # packed fp32 VALU forms are kept out of the generated code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libwsl)")


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(hipcc: str, src: str, verbose: bool) -> str:
    obj = os.path.join(BUILD_DIR, os.path.basename(src)[:-4] + ".o")
    cmd = [hipcc, *HIPCC_FLAGS, f"-I{INCLUDE_DIR}", f"-I{CSRC}", "-c", src, "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{res.stdout}\n{res.stderr}")
    return obj


def _stale(src: str) -> bool:
    """Whether src's object is missing or older than src or any header it may include."""
    obj = os.path.join(BUILD_DIR, os.path.basename(src)[:-4] + ".o")
    if not os.path.exists(obj):
        return True
    deps = [src] + [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".h")] + \
           [os.path.join(INCLUDE_DIR, f) for f in os.listdir(INCLUDE_DIR) if f.endswith(".h")]
    return max(os.path.getmtime(d) for d in deps) > os.path.getmtime(obj)


def build_library(verbose: bool = False, jobs: int | None = None, incremental: bool = False) -> str:
    """Compiles every csrc/*.hip and links libwsl.so. Rebuilds everything unless
    `incremental`, which recompiles only sources whose object is out of date."""
    hipcc = _hipcc()
    os.makedirs(BUILD_DIR, exist_ok=True)
    srcs = sources()
    todo = [s for s in srcs if _stale(s)] if incremental else srcs
    jobs = jobs or min(max(len(todo), 1), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda s: _compile(hipcc, s, verbose), todo))
    objs = [os.path.join(BUILD_DIR, os.path.basename(s)[:-4] + ".o") for s in srcs]
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


STAMPS_LIB_PATH = os.path.join(PKG_DIR, "libwsl_stamps.so")
TEMPORAL_LIB_PATH = os.path.join(PKG_DIR, "libwsl_temporal.so")


def _variant_library(define: str, names: tuple, suffix: str, out: str, verbose: bool) -> str:
    """libwsl with the sources `names` compiled with -D`define` (objects `<name>_<suffix>.o`)
    and the other objects of the last ``build_library``; the product library is left as it is."""
    hipcc = _hipcc()
    if not os.path.exists(LIB_PATH):
        build_library(verbose=verbose)

    def compiled(name: str) -> str:
        src = os.path.join(CSRC, name)
        obj = os.path.join(BUILD_DIR, name[:-4] + f"_{suffix}.o")
        cmd = [hipcc, *HIPCC_FLAGS, f"-D{define}", f"-I{INCLUDE_DIR}", f"-I{CSRC}", "-c", src, "-o", obj]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src}:\n{res.stdout}\n{res.stderr}")
        return obj

    with ThreadPoolExecutor(max_workers=len(names)) as ex:
        variant_objs = list(ex.map(compiled, names))
    objs = [os.path.join(BUILD_DIR, os.path.basename(s)[:-4] + ".o") for s in sources()
            if os.path.basename(s) not in names] + variant_objs
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", out]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    return out


def build_stamps_library(verbose: bool = False) -> str:
    """libwsl_stamps.so: libwsl with the prefill and decode kernels built with -DWSL_STAMPS
    (per-phase wall-clock stamps of every workgroup, read back by ``wsl_prefill_stamps`` and
    ``wsl_decode_stamps``), for ``bench.py --only stamps`` run with WSL_LIB pointing at it."""
    return _variant_library("WSL_STAMPS", ("lora_prefill.hip", "lora_decode.hip"), "stamps", STAMPS_LIB_PATH,
                            verbose)


def build_temporal_library(verbose: bool = False) -> str:
    """libwsl_temporal.so: libwsl with the prefill kernel's output stores through the caches
    (-DWSL_TEMPORAL_STORES) instead of non-temporal, for side-by-side timing with WSL_LIB
    pointing at it."""
    return _variant_library("WSL_TEMPORAL_STORES", ("lora_prefill.hip",), "temporal", TEMPORAL_LIB_PATH, verbose)


if __name__ == "__main__":
    if "--stamps" in sys.argv:
        print(build_stamps_library(verbose="-v" in sys.argv))
    elif "--temporal-stores" in sys.argv:
        print(build_temporal_library(verbose="-v" in sys.argv))
    else:
        path = build_library(verbose="-v" in sys.argv, incremental="--incremental" in sys.argv)
        print(path)
