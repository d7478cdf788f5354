"""Builds libmaxuna_moe.so (gfx950) in-tree with hipcc.

    python -m maxuna_amd.build          # compile every source, link the library

The library lands in maxuna_amd/lib/ so it travels with the source tree; it is
git-ignored.  Compilation always runs (no staleness check): the caller decides
when to build.
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
LIB_DIR = PKG / "lib"
LIB_NAME = "libmaxuna_moe.so"
SOURCES = ["mx_api.hip", "mx_dequant.hip", "mx_mv.hip", "mx_mvf.hip", "mx_route.hip", "mx_elem.hip", "mx_mm.hip", "mx_gemm.hip", "mx_vmm.hip",
           "mx_gguf.cpp"]
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    # every product/difference is rounded on its own unless written as an fma
    "-ffp-contract=off",
    # no packed-FP32 VALU ops anywhere in device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build maxuna_moe)")


def _compile(src: str, obj_dir: Path) -> Path:
    obj = obj_dir / (Path(src).stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{proc.stderr}")
    # the host pass does not know the GPU-only feature flag; everything else is shown
    noise = "'-packed-fp32-ops' is not a recognized feature"
    rest = [ln for ln in proc.stderr.splitlines() if noise not in ln and ln.strip()]
    if rest:
        sys.stderr.write(f"[{src}]\n" + "\n".join(rest) + "\n")
    return obj


def build(verbose: bool = True) -> Path:
    obj_dir = LIB_DIR / "obj"
    obj_dir.mkdir(parents=True, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4)) as ex:
        objs = list(ex.map(lambda s: _compile(s, obj_dir), SOURCES))
    out = LIB_DIR / LIB_NAME
    tmp = LIB_DIR / (LIB_NAME + ".tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    # every symbol must resolve (a kernel the host pass dropped leaves its launch
    # stub undefined, which only the dynamic loader reports)
    import ctypes
    ctypes.CDLL(os.fspath(tmp), mode=os.RTLD_NOW)
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    build()
