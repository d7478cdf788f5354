"""No kernel of the built library keeps data in scratch (private) memory.

A register array indexed by a value the compiler cannot resolve, a lambda it
declines to inline, or a register budget too small for the kernel all move
data to scratch, and every such access becomes a memory round trip: two such
kernels ran 10-36x slower with correct results.  This reads the gfx950 code
objects this build produced (maxuna_amd/lib/obj/*.o: the offload bundle in
each object's .hip_fatbin section) and checks every kernel's
.private_segment_fixed_size.
"""
import re
import subprocess
from pathlib import Path

import pytest

from maxuna_amd import build as B

LLVM = Path("/opt/rocm/llvm/bin")
TARGET = f"hipv4-amdgcn-amd-amdhsa--{B.ARCH}"
# (kernel symbol, bytes): register spills the kernel's budget cannot avoid
ALLOWED = {
    # plain Q4_K GEMM, full-tile and FEW forms: 2-3 VGPRs at the 256 cap, stored
    # before the K loop and reloaded after it
    "_ZN2mx12_GLOBAL__N_16k_gemmILi12ELb0ELb0EEEvNS_8GemmArgsE": 12,
    "_ZN2mx12_GLOBAL__N_16k_gemmILi12ELb0ELb1EEEvNS_8GemmArgsE": 8,
}


def _kernels(obj: Path, tmp: Path):
    fat, co = tmp / (obj.stem + ".fat"), tmp / (obj.stem + ".co")
    r = subprocess.run([str(LLVM / "llvm-objcopy"), f"--dump-section=.hip_fatbin={fat}", str(obj), str(tmp / "x.o")],
                       capture_output=True, text=True)
    if r.returncode:  # no device code in this object
        return {}
    subprocess.run([str(LLVM / "clang-offload-bundler"), "--unbundle", "--type=o", f"--input={fat}",
                    f"--targets={TARGET}", f"--output={co}"], check=True, capture_output=True)
    notes = subprocess.run([str(LLVM / "llvm-readelf"), "--notes", str(co)], check=True, capture_output=True,
                           text=True).stdout
    names = re.findall(r"^\s+\.name:\s+(\S+)", notes, re.M)
    sizes = [int(v) for v in re.findall(r"\.private_segment_fixed_size:\s+(\d+)", notes)]
    assert len(names) == len(sizes), f"{obj.name}: kernel metadata not understood"
    return dict(zip(names, sizes))


def test_no_kernel_uses_scratch(tmp_path):
    objs = sorted((B.LIB_DIR / "obj").glob("*.o"))
    if not objs or not all((LLVM / t).exists() for t in ("llvm-objcopy", "clang-offload-bundler", "llvm-readelf")):
        pytest.skip("library objects or LLVM tools not present (run build() first)")
    found, bad = 0, []
    for obj in objs:
        for name, size in _kernels(obj, tmp_path).items():
            found += 1
            if size > ALLOWED.get(name, 0):
                bad.append(f"{obj.name}: {name} uses {size} bytes of scratch per lane")
    assert found > 100, f"only {found} kernels found"
    assert not bad, "\n".join(bad)
