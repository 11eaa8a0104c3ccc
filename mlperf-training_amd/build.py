"""Ahead-of-time build of the HIP kernels into one C-ABI shared library.

    python mlperf-training_amd/build.py        # -> hstu_amd/libhstu_mi355x.so

hipcc cross-compiles for gfx950 without a GPU.  Each source compiles to its
own object in parallel (``_build/``), then one link makes the library.  The
library links only the HIP runtime (no torch symbols), so any FFI (ctypes
here) can bind it.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
REPO_ROOT = PKG_ROOT.parent
CSRC = PKG_ROOT / "csrc"
OBJ_DIR = PKG_ROOT / "_build"
OUT = PKG_ROOT / "hstu_amd" / "libhstu_mi355x.so"
SOURCES = ["hstu_attention.hip", "hstu_fp8_gemm.hip", "hstu_layernorm.hip", "hstu_delta.hip", "hstu_do_fp8.hip",
           "hstu_wgrad.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # no packed-FP32 VALU ops anywhere in device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return str(Path(rocm) / "bin" / "hipcc")


def _run(cmd, verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed ({res.returncode}): {cmd[-1]}")


def build(verbose: bool = False, jobs: int = 0) -> Path:
    srcs = [CSRC / s for s in SOURCES if (CSRC / s).exists()]
    OBJ_DIR.mkdir(exist_ok=True)
    objs = [OBJ_DIR / (s.stem + ".o") for s in srcs]
    inc = f"-I{REPO_ROOT / 'include'}"
    jobs = jobs or min(len(srcs), max(1, os.cpu_count() or 1), 16)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_run, [hipcc(), *HIPCC_FLAGS, inc, "-c", str(s), "-o", str(o)], verbose)
                for s, o in zip(srcs, objs)]
        for f in futs:
            f.result()
    tmp = OUT.with_suffix(".so.tmp")
    _run([hipcc(), "--offload-arch=gfx950", "-shared", *map(str, objs), "-o", str(tmp)], verbose)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
