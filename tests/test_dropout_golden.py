"""Dropout masks against the reference's own kernels.

``tests/golden/dropout_masks.npz`` holds masks that the reference's Triton
kernels ``_generate_random_mask`` / ``_generate_random_mask16``
(recommendation_v4/hstu/generative_recommenders/ops/triton/
triton_hstu_linear.py:331-375, 428-470) produced under Triton's CPU
interpreter (``tests/golden/make_dropout_masks.py``): ragged row counts for
both row groupings, ragged D, 1-3 masks, p = 0 and a 64-bit seed.  The CPU
test pins the oracle's counter layout to them bitwise; the GPU test checks
the HIP mask kernel bitwise at the D values it serves."""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import hstu_ln_oracle as L

GOLDEN = Path(__file__).parent / "golden" / "dropout_masks.npz"


def _cases():
    z = np.load(GOLDEN)
    for i, ((N, D, nm, seed), p) in enumerate(zip(z["int_params"], z["p"])):
        yield i, int(N), int(D), int(nm), float(p), int(seed), z[f"mask32_{i}"], z[f"mask16_{i}"]


def test_oracle_masks_match_reference_kernels():
    n = 0
    for i, N, D, nm, p, seed, m32, m16 in _cases():
        for mask16, want in ((False, m32), (True, m16)):
            got = L.dropout_mask_rows(np.arange(N), D, nm, p, seed, mask16)
            assert np.array_equal(got, want), f"case {i} mask16={mask16}"
            n += 1
    assert n == 10


@pytest.mark.gpu
def test_gpu_masks_match_reference_kernels(hip_lib):
    import hstu_amd
    from hstu_amd.hstu_linear import SERVED_D

    served = 0
    for i, N, D, nm, p, seed, m32, m16 in _cases():
        if D not in SERVED_D:
            continue
        concat_u, concat_x = nm >= 2, nm >= 3
        for mask16, want in ((False, m32), (True, m16)):
            print(f"dropout mask case {i}: N={N} D={D} masks={nm} mask16={mask16}", flush=True)
            got = hstu_amd.create_dropout_mask(N, D, concat_u, concat_x, p, seed, "cuda", mask16=mask16)
            assert np.array_equal(got.cpu().numpy(), want), f"case {i} mask16={mask16}"
            served += 1
    assert served >= 4
