"""Build libhclsm_amd.so (all HIP sources under csrc/) for gfx950 with hipcc.

Usage:  python -m hclsm_amd.build        (or hclsm_amd.build.build() from Python)

The library lands in ``hclsm_amd/_lib/libhclsm_amd.so`` inside the source tree so
that it travels with the repository snapshot to the GPU box.  Objects are built in
parallel into ``hclsm_amd/_lib/obj`` and linked with ``hipcc -shared``.
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
LIBDIR = PKG / "_lib"
LIBNAME = "libhclsm_amd.so"
ARCH = "gfx950"

# -packed-fp32-ops: keep the compiler from forming v_pk_{add,mul,fma}_f32.
HIPCC_FLAGS = [
    "-O3", "-std=c++20", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-gpu-rdc", "-Wno-unused-result",
]

# Per-source extras.  The scan keeps its MFMA accumulator in the VGPRs it also updates with
# VALU ops every step; the VGPR form of MFMA avoids an AGPR<->VGPR copy of all 16 states.
FILE_FLAGS = {
    "ssm_scan.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    # The attention's score and output tiles are consumed by VALU code right after each MFMA; in the VGPR
    # form they need no AGPR copies and the kernel takes fewer registers (more waves per SIMD).
    "event_attn.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the hclsm_amd kernels need ROCm's hipcc to build")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def lib_path() -> Path:
    return LIBDIR / LIBNAME


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every csrc/*.hip and link the shared library; returns its path."""
    hipcc = _hipcc()
    objdir = LIBDIR / "obj"
    objdir.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")

    def compile_one(src: Path) -> Path:
        obj = objdir / (src.stem + ".o")
        cmd = [hipcc, *HIPCC_FLAGS, *FILE_FLAGS.get(src.name, []), "-I", str(PKG.parent / "include"), "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src.name}:\n{r.stderr[-8000:]}")
        return obj

    jobs = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, srcs))
    out = lib_path()
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-8000:]}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    p = build(verbose="-v" in sys.argv)
    print(p)
