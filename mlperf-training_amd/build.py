"""Ahead-of-time build of the HIP kernels into one C-ABI shared library.

    python mlperf-training_amd/build.py        # -> hstu_amd/libhstu_mi355x.so

hipcc cross-compiles for gfx950 without a GPU.  The library links only the
HIP runtime (no torch symbols), so any FFI (ctypes here) can bind it.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
REPO_ROOT = PKG_ROOT.parent
CSRC = PKG_ROOT / "csrc"
OUT = PKG_ROOT / "hstu_amd" / "libhstu_mi355x.so"
SOURCES = ["hstu_attention.hip", "hstu_fp8_gemm.hip", "hstu_layernorm.hip", "hstu_delta.hip", "hstu_do_fp8.hip",
           "hstu_wgrad.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # no packed-FP32 VALU ops anywhere in device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return str(Path(rocm) / "bin" / "hipcc")


def build(verbose: bool = False) -> Path:
    srcs = [str(CSRC / s) for s in SOURCES if (CSRC / s).exists()]
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{REPO_ROOT / 'include'}", *srcs, "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed ({res.returncode})")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
