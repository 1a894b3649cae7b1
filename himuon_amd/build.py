"""Build libhimuon_hip.so (gfx950) in-tree with hipcc.

Usage: ``python -m himuon_amd.build`` (or ``__graft_entry__.build()``).
The library is written to ``himuon_amd/lib/libhimuon_hip.so``; the HIP
sources are compiled in parallel, one object per source, then linked.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIBDIR = PKG / "lib"
LIB = LIBDIR / "libhimuon_hip.so"
SOURCES = ["tile_io.hip", "apply.hip", "adamw.hip", "ns5.hip", "ns5_stream.hip", "ns5_lds.hip", "ns5_ba.hip", "ns5_small.hip", "products.hip", "capi.hip"]
ARCH = os.environ.get("HIMUON_OFFLOAD_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Packed fp32 VALU ops are kept out of the generated code.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")


def build_library(verbose: bool = False) -> Path:
    """Compile every HIP source and link libhimuon_hip.so. Always rebuilds."""
    objdir = LIBDIR / "obj"
    objdir.mkdir(parents=True, exist_ok=True)
    srcs = [CSRC / s for s in SOURCES]
    objs = [objdir / (s.stem + ".o") for s in srcs]

    def compile_one(pair):
        src, obj = pair
        cmd = [HIPCC, *COMMON_FLAGS, "-I", str(PKG.parent / "include"), "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        _run(cmd)

    with ThreadPoolExecutor(max_workers=min(len(srcs), os.cpu_count() or 1)) as ex:
        list(ex.map(compile_one, zip(srcs, objs)))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    _run(cmd)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    path = build_library(verbose="-v" in sys.argv)
    print(path)
