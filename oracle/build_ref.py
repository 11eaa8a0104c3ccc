"""Builds the reference's own K=512 FP8 GEMM from its source, where it lies,
into ``oracle/_ref/`` -- TEST INFRASTRUCTURE ONLY: the library is a checker
for ``tests/test_k512_ref_gpu.py`` and is never loaded by the product.

    python oracle/build_ref.py        # needs /root/reference (this container)

Source: ``recommendation_v4/hstu/generative_recommenders/ops/hip/k512_fp8_gemm.cu``
(it includes only <hip/hip_runtime.h>), compiled as its header's build line
states (``-DKITTENS_CDNA4 -std=c++20 -O3 -DHK_N={1536|1024} -ffp-contract=off``)
with this repository's gfx950 flags added (no packed-FP32 VALU code).  The
output, ``oracle/_ref/libk512_fp8_gemm_n{N}.so``, exports
``k512_fp8_gemm_e4m3_bias_N{N}(A, B, C, bias, sa, sb, M, stream)``.  Nothing
from the reference is copied into the repository; the built file is
git-ignored and travels to the GPU box with the tree.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

REF = Path("/root/reference/recommendation_v4/hstu/generative_recommenders/ops/hip/k512_fp8_gemm.cu")
OUT_DIR = Path(__file__).resolve().parent / "_ref"
WIDTHS = (1536,)


def build(verbose: bool = False) -> list:
    """The libraries built (empty when the reference tree is absent)."""
    if not REF.exists():
        if verbose:
            print(f"oracle/_ref: {REF} absent; nothing built")
        return []
    OUT_DIR.mkdir(exist_ok=True)
    hipcc = str(Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "bin" / "hipcc")
    built = []
    for n in WIDTHS:
        out = OUT_DIR / f"libk512_fp8_gemm_n{n}.so"
        cmd = [hipcc, "-DKITTENS_CDNA4", "--offload-arch=gfx950", "-std=c++20", "-O3", f"-DHK_N={n}",
               "-mllvm", "-amdgpu-sched-strategy=iterative-ilp", "-ffp-contract=off",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               "-shared", "-fPIC", str(REF), "-o", str(out)]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            sys.stderr.write(res.stdout + res.stderr)
            raise RuntimeError(f"reference build failed: {out.name}")
        built.append(out)
    return built


if __name__ == "__main__":
    print(build(verbose=True))
