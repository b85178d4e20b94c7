"""Build the HIP library ``multics_amd/_lib/libhierattn.so`` for gfx950.

One ``hipcc`` invocation over ``multics_amd/csrc/*.hip``; no torch extension,
no CMake.  Packed-FP32 instruction selection (v_pk_*_f32) is disabled for
every device translation unit because some of its forms have produced silent
wrong results on the target machines; the host pass warns that it does not
know the feature, which is harmless.  ``-fno-honor-nans`` lets fmax compile to
plain v_max / v_max3 without NaN canonicalisation (infinities are still
honoured: masked scores are -inf).
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
LIB = LIB_DIR / "libhierattn.so"
ARCH = os.environ.get("HIERATTN_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC)")


def build(verbose: bool = False) -> Path:
    LIB_DIR.mkdir(exist_ok=True)
    sources = sorted(str(p) for p in CSRC.glob("*.hip"))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
           "-fno-honor-nans",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           f"-I{ROOT / 'include'}", f"-I{CSRC}", *sources, "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{errs}")
    if verbose and errs.strip():
        print(errs, file=sys.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
