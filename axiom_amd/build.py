"""Build the gfx950 KDA library in-tree: ``axiom_amd/libkda_mi355x.so``.

Every HIP source under ``axiom_amd/csrc`` is compiled with hipcc for gfx950
only, then linked into one shared library whose exported symbols are exactly
the C ABI of ``include/kda_mi355x.h``.  Run ``python -m axiom_amd.build`` or
call :func:`build`.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libkda_mi355x.so"
INCLUDE = PKG.parent / "include"

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    # packed fp32 VALU ops are kept out of every kernel of this library
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]
SOURCES = ["kda_chunk.hip", "kda_varlen.hip", "kda_decode.hip", "kda_bwd.hip", "kda_ut.hip", "kda_prologue.hip", "kda_api.hip"]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the KDA library needs ROCm's hipcc to build")


def _compile(src: Path, obj: Path, hipcc: str) -> None:
    cmd = [hipcc, *HIPCC_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{p.stderr}")


def build(verbose: bool = False) -> Path:
    """Compile all sources and link ``libkda_mi355x.so``; returns its path."""
    hipcc = _hipcc()
    BUILD.mkdir(exist_ok=True)
    objs = [BUILD / (s.replace(".hip", ".o")) for s in SOURCES]
    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 1)) as ex:
        list(ex.map(lambda so: _compile(CSRC / so[0], so[1], hipcc), zip(SOURCES, objs)))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"link failed:\n{p.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
