"""Build the gfx950 HIP library ``libgfx906_fa_amd.so`` in place.

    python gfx906-fa-vllm_amd/build.py

One hipcc invocation over csrc/*.hip (plain C ABI, no torch headers), so the
library is independent of the PyTorch build and is loaded with ctypes.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB_NAME = "libgfx906_fa_amd.so"
SOURCES = ["q8_quant.hip", "q8_rope.hip", "q8_gather.hip", "q8_pack.hip", "paged_attn.hip", "hbm_probe.hip"]
ARCH = os.environ.get("GFX906_FA_AMD_ARCH", "gfx950")


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc"):
        if c and os.path.exists(c):
            return c
    return "hipcc"


def build(verbose: bool = False, out: str | None = None, defines=()) -> str:
    """Compiles csrc/*.hip into `out` (default: the in-tree library).
    `defines`: extra -D tuning macros (GFA_DEC_DEPTH, GFA_DEC_RING, GFA_PF_PDEPTH, ...: the
    `#ifndef GFA_*` defaults in csrc/)."""
    out = out or os.path.join(HERE, LIB_NAME)
    tmp = out + ".tmp"
    cmd = [
        hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
        # no fast-math: the Q8_0 quantizer needs IEEE division and rint
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", os.path.join(ROOT, "include"), "-I", os.path.join(HERE, "csrc"),
        *[f"-D{d}" for d in defines],
        *[os.path.join(HERE, "csrc", s) for s in SOURCES],
        "-o", tmp,
    ]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(l for l in (res.stderr or "").splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{errs}")
    if verbose and errs.strip():
        print(errs)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
