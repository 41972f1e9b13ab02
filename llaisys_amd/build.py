"""Build libllaisys.so (HIP, gfx950) in-tree.

Compiles every source under llaisys_amd/csrc with hipcc for gfx950 into
llaisys_amd/_build/ and links llaisys_amd/libllaisys/libllaisys.so, the
library the ctypes layer loads (the reference loads libllaisys.so from its
package dir the same way, python/llaisys/libllaisys/__init__.py:17-40).

Run: python llaisys_amd/build.py   (or __graft_entry__.build()).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "libllaisys" / "libllaisys.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

COMMON = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    f"--offload-arch={ARCH}",
    f"-I{ROOT / 'include'}",
    # Packed fp32 VALU ops are disabled for every HIP compile on this hardware.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fvisibility=hidden",
]


# Per-source extra flags. gemm.hip: keep MFMA accumulators in VGPRs (the
# AGPR form of the gfx950 16x16x32 MFMAs makes the register allocator rotate
# the loop-carried accumulators through v_accvgpr copies every k step).
EXTRA = {
    "kernels/gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _sources() -> list[Path]:
    return sorted(p for p in CSRC.rglob("*") if p.suffix in (".cpp", ".hip"))


def _compile(src: Path) -> Path:
    rel = src.relative_to(CSRC)
    obj = OBJ / (str(rel).replace(os.sep, "__") + ".o")
    cmd = [HIPCC, *COMMON, *EXTRA.get(rel.as_posix(), []), "-c", str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd[1:1] = ["-x", "hip"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {rel}:\n{r.stderr}")
    return obj


def build(verbose: bool = True) -> Path:
    """Compile all HIP/C++ sources and link the shared library. Always rebuilds."""
    OBJ.mkdir(exist_ok=True)
    srcs = _sources()
    jobs = int(os.environ.get("MAX_JOBS", "8"))
    with cf.ThreadPoolExecutor(max_workers=max(1, min(jobs, 16))) as ex:
        objs = list(ex.map(_compile, srcs))
    LIB.parent.mkdir(exist_ok=True)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"[llaisys_amd.build] {len(srcs)} sources -> {LIB.relative_to(ROOT)}")
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
