"""Write tests/golden/dropout_masks.npz: dropout masks from the reference's
own Triton kernels, run under Triton's CPU interpreter in the build container.

Run from the repository root (needs /root/reference, Triton and torch):

    python tests/golden/make_dropout_masks.py

Reference kernels (recommendation_v4/hstu/generative_recommenders/):
``ops/triton/triton_hstu_linear.py`` ``_generate_random_mask`` (:331-375,
32-bit keep test, 4 rows per Philox call) and ``_generate_random_mask16``
(:428-470, 16-bit halves, 8 rows per call), launched the way
``_create_dropout_mask`` (:2547-2598) launches them: grid cdiv(N, 4) / cdiv(N,
8), BLOCK_D = next power of two >= D, NUM_MASKS = 1 + concat_u + concat_x,
thresholds from ``_mask_keep_above`` / ``_mask_keep_min16``.

The fixture holds inputs and outputs only: per case (N, D, num_masks, p,
seed) and the [N, D] int8 masks of both schemes.
"""

import os
import sys
from pathlib import Path

os.environ["TRITON_INTERPRET"] = "1"  # before triton is imported

import numpy as np  # noqa: E402
import torch  # noqa: E402

REF = "/root/reference/recommendation_v4/hstu"
OUT = Path(__file__).with_name("dropout_masks.npz")

# (N, D, num_masks, p, seed): ragged N for both row groupings, ragged D
# (BLOCK_D > D), 1 / 2 / 3 masks, p = 0 (keep all), a 64-bit seed
CASES = [
    (19, 64, 3, 0.3, 12345),
    (37, 512, 3, 0.1, 2**61 + 12345),
    (8, 100, 2, 0.5, 7),
    (13, 512, 1, 0.0, 99),
    (21, 192, 3, 0.3, 2**40 + 3),
]


def main() -> None:
    sys.path.insert(0, REF)
    import triton
    from generative_recommenders.ops.triton import triton_hstu_linear as ref

    arrays = {}
    params = []
    for i, (N, D, nm, p, seed) in enumerate(CASES):
        bd = triton.next_power_of_2(D)
        m32 = torch.empty(N, D, dtype=torch.int8)
        ref._generate_random_mask[(triton.cdiv(N, 4),)](m32, N, ref._mask_keep_above(p), seed, D, m32.stride(0),
                                                        bd, nm)
        m16 = torch.empty(N, D, dtype=torch.int8)
        ref._generate_random_mask16[(triton.cdiv(N, 8),)](m16, N, ref._mask_keep_min16(p), seed, D,
                                                          m16.stride(0), bd, nm)
        arrays[f"mask32_{i}"] = m32.numpy()
        arrays[f"mask16_{i}"] = m16.numpy()
        params.append((N, D, nm, seed))
        print(f"case {i}: N={N} D={D} masks={nm} p={p} seed={seed}", flush=True)
    arrays["int_params"] = np.array(params, dtype=np.int64)  # N, D, num_masks, seed
    arrays["p"] = np.array([c[3] for c in CASES], dtype=np.float64)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
