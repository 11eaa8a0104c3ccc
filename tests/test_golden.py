"""The oracle's mask (and the scalar form the kernels' mask follows) against
masks written by the reference's own ``_get_valid_attn_mask``
(tests/golden/valid_attn_mask.npz, made by tests/golden/make_mask_golden.py)."""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import hstu_oracle as orc

GOLDEN = np.load(Path(__file__).parent / "golden" / "valid_attn_mask.npz")
CASES = sorted({k.split("__")[0] for k in GOLDEN.files})


def _case(name):
    N, mal, ctx, mfull = (int(x) for x in GOLDEN[f"{name}__args"])
    lengths = torch.tensor(GOLDEN[f"{name}__lengths"])
    nt = GOLDEN[f"{name}__num_targets"]
    nt = torch.tensor(nt) if nt.size else None
    return N, lengths, nt, mal, ctx, mfull, torch.tensor(GOLDEN[f"{name}__mask"])


@pytest.mark.parametrize("name", CASES)
def test_oracle_mask_matches_reference(name):
    N, lengths, nt, mal, ctx, mfull, want = _case(name)
    got = orc.valid_attn_mask(N, lengths, nt, mal, ctx, mfull)
    assert torch.equal(got.expand_as(want), want)


@pytest.mark.parametrize("name", [c for c in CASES if not c.endswith("_full")])
def test_scalar_mask_matches_reference(name):
    """valid_pair is the per-element predicate the HIP kernels evaluate."""
    N, lengths, nt, mal, ctx, _, want = _case(name)
    for b, L in enumerate(lengths.tolist()):
        for i in range(L):
            for j in range(L):
                ntb = None if nt is None else int(nt[b])
                assert orc.valid_pair(i, j, L, ntb, mal, ctx) == bool(want[b if want.shape[0] > 1 else 0, i, j])


@pytest.mark.parametrize("name", CASES)
def test_pytorch_backend_mask_matches_reference(name):
    from hstu_amd.pt_hstu_attention import get_valid_attn_mask

    N, lengths, nt, mal, ctx, mfull, want = _case(name)
    got = get_valid_attn_mask(torch.device("cpu"), True, N, lengths, nt, mal, ctx, mfull)
    assert torch.equal(got.expand_as(want), want)
