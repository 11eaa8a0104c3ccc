"""Writes tests/golden/valid_attn_mask.npz: masks produced by the reference's
own ``_get_valid_attn_mask`` (recommendation_v4/hstu/generative_recommenders/
ops/pytorch/pt_hstu_attention.py:32-84) for the non-production mask options
(num_targets > 1, contextual_seq_len, max_attn_len with and without
min_full_attn_seq_len), which no closed form in tests/test_oracle.py pins.

Run in the build container only (the reference is not present on the GPU box):
    python tests/golden/make_mask_golden.py /root/reference
The fixture holds inputs and outputs only.
"""

import importlib.util
import sys
from pathlib import Path

import numpy as np
import torch

CASES = [
    # name, N, lengths, num_targets, max_attn_len, contextual_seq_len, min_full_attn_seq_len
    ("targets", 12, [12, 9, 5], [3, 1, 2], 0, 0, 0),
    ("contextual", 12, [12, 7], None, 0, 3, 0),
    ("max_attn_len", 12, [12, 10], None, 4, 0, 0),
    ("max_attn_len_full", 12, [12, 10], None, 4, 0, 3),
    ("all", 14, [14, 11, 6], [2, 3, 1], 5, 2, 0),
    ("all_full", 14, [14, 11, 6], [2, 3, 1], 5, 2, 2),
]


def main(ref_root: str) -> None:
    path = Path(ref_root) / "recommendation_v4/hstu/generative_recommenders/ops/pytorch/pt_hstu_attention.py"
    spec = importlib.util.spec_from_file_location("ref_pt_hstu_attention", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    out = {}
    for name, N, lengths, nt, mal, ctx, mfull in CASES:
        m = mod._get_valid_attn_mask(
            device=torch.device("cpu"), causal=True, N=N, seq_lengths=torch.tensor(lengths),
            num_targets=None if nt is None else torch.tensor(nt), max_attn_len=mal,
            contextual_seq_len=ctx, min_full_attn_seq_len=mfull)
        out[f"{name}__mask"] = m.numpy()
        out[f"{name}__args"] = np.array([N, mal, ctx, mfull], dtype=np.int64)
        out[f"{name}__lengths"] = np.array(lengths, dtype=np.int64)
        out[f"{name}__num_targets"] = np.array(nt if nt is not None else [], dtype=np.int64)
    dst = Path(__file__).resolve().parent / "valid_attn_mask.npz"
    np.savez_compressed(dst, **out)
    print(dst, len(CASES), "cases")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
