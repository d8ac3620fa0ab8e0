"""Builds libxk_moe.so (all HIP sources under csrc/) for gfx950 with hipcc.

Usage: ``python -m xkernels_amd.build`` (or ``__graft_entry__.build()``). The
library lands in ``xkernels_amd/_lib/`` inside the source tree so it travels
with the repository to the GPU host.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB_DIR = PKG / "_lib"
LIB = LIB_DIR / "libxk_moe.so"
ARCH = "gfx950"

SOURCES = ["capi.hip", "align.hip", "reduce.hip", "int4_gemm.hip", "int4_stream.hip", "int4_prefill.hip", "mxfp4_gemm.hip", "topk_softmax.hip"]

# Packed-fp32 VALU ops are disabled for every device pass: the compiler must not
# form v_pk_{add,mul,fma}_f32 from float code.
HIPFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def build(verbose: bool = False) -> Path:
    """Compile every source to an object, then link the shared library."""
    LIB_DIR.mkdir(exist_ok=True)
    obj_dir = PKG / "_build"
    obj_dir.mkdir(exist_ok=True)
    cc = hipcc()
    objs = []
    procs = []
    for src in SOURCES:
        obj = obj_dir / (Path(src).stem + ".o")
        cmd = [cc, *HIPFLAGS, "-I", str(ROOT / "include"), "-c", str(CSRC / src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
        objs.append(str(obj))
    failed = []
    for src, p in procs:
        out, _ = p.communicate()
        # the host pass does not know the device-only feature; that note is noise
        lines = [ln for ln in out.splitlines() if "packed-fp32-ops" not in ln]
        if lines and (verbose or p.returncode):
            print("\n".join(lines), file=sys.stderr)
        if p.returncode:
            failed.append(src)
    if failed:
        raise RuntimeError(f"hipcc failed for {failed}")
    tmp = LIB.with_suffix(".so.tmp")
    link = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", str(tmp)]
    subprocess.run(link, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
