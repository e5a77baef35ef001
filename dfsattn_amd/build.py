"""Builds libdfsattn_amd.so (all HIP kernels + the C-ABI) for gfx950 in-tree.

Run ``python -m dfsattn_amd.build`` or call :func:`build`. The library lands in
``dfsattn_amd/_lib/`` so it travels with the source tree.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
INCLUDE = os.path.join(REPO_DIR, "include")
OUT_DIR = os.path.join(PKG_DIR, "_lib")
LIB_NAME = "libdfsattn_amd.so"
SOURCES = ["host.cpp", "permute.hip", "score_topk.hip", "bsa_fwd.hip", "masks.hip", "norm_rope.hip", "dit_fused.hip"]
ARCH = "gfx950"


def _hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = os.path.join(rocm, "bin", "hipcc")
    return cand if os.path.exists(cand) else (shutil.which("hipcc") or "hipcc")


def _flags() -> list:
    return [
        "-O3",
        "-std=c++17",
        "-fPIC",
        f"--offload-arch={ARCH}",
        # Packed-FP32 VALU forms stay disabled in every kernel.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", INCLUDE,
        "-I", CSRC,
        "-Wno-unused-result",
    ]


def build(verbose: bool = False, jobs: int = 8) -> str:
    """Compiles every source to an object in _lib/obj and links the .so."""
    hipcc = _hipcc()
    obj_dir = os.path.join(OUT_DIR, "obj")
    os.makedirs(obj_dir, exist_ok=True)

    def compile_one(src: str) -> str:
        obj = os.path.join(obj_dir, src + ".o")
        path = os.path.join(CSRC, src)
        lang = ["-x", "hip"] if src.endswith(".hip") else []
        cmd = [hipcc, *_flags(), *lang, "-c", path, "-o", obj]
        res = subprocess.run(cmd, capture_output=True, text=True)
        out = (res.stdout + res.stderr).strip()
        noise = "is not a recognized feature for this target"
        shown = "\n".join(l for l in out.splitlines() if noise not in l)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src}:\n{shown}")
        if verbose and shown:
            print(shown, file=sys.stderr)
        return obj

    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    lib = os.path.join(OUT_DIR, LIB_NAME)
    tmp = lib + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}{res.stderr}")
    os.replace(tmp, lib)
    return lib


if __name__ == "__main__":
    print(build(verbose=True))
