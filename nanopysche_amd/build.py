"""Build recipe for libfm_hip.so (gfx950), in-tree next to this file.

    python -m nanopysche_amd.build          # or __graft_entry__.build()

Each translation unit is compiled by hipcc for gfx950 only, in parallel, then
linked into one shared library.  Packed fp32 instructions are disabled
(``-packed-fp32-ops``) for every device compile.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libfm_hip.so"
SOURCES = ["fm_api.cpp", "fm_quant.hip", "fm_route.hip", "fm_swiglu.hip", "fm_gemm.hip", "fm_router.hip",
           "fm_norm.hip"]
ARCH = "gfx950"


def source_hash() -> str:
    """Hash of every file the library is built from (csrc/ and include/); the
    build stamps it into libfm_hip.so and the loader refuses a library whose
    stamp differs from the sources beside it."""
    import hashlib

    h = hashlib.sha256()
    files = sorted([*CSRC.glob("*.hip"), *CSRC.glob("*.h"), *CSRC.glob("*.cpp"),
                    *(PKG.parent / "include").glob("*.h")])
    for f in files:
        h.update(f.name.encode())
        h.update(b"\0")
        h.update(f.read_bytes())
    return h.hexdigest()[:16]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libfm_hip.so)")


def _flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-Wall",
        "-Wno-unused-result",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    ]


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    hipcc = _hipcc()
    obj_dir = PKG / "_build"
    obj_dir.mkdir(exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 4, 16)

    stamp = source_hash()

    def compile_one(src: str) -> Path:
        obj = obj_dir / (src.replace(".", "_") + ".o")
        lang = ["-x", "hip"] if src.endswith(".hip") else []
        extra = [f'-DFM_SOURCE_HASH="{stamp}"'] if src == "fm_api.cpp" else []
        cmd = [hipcc, *_flags(), *extra, *lang, "-c", str(CSRC / src), "-o", str(obj)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
        if verbose and r.stderr.strip():
            print(r.stderr, file=sys.stderr)
        return obj

    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
