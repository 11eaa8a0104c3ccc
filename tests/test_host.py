"""Host-side logic on the CPU: shape policy and fallible entry points, the
PYTORCH backend against the oracle, bench CLI guard."""

import subprocess
import sys
from pathlib import Path

import pytest
import torch

from oracle import hstu_oracle as orc

REPO = Path(__file__).resolve().parents[1]


def test_unsupported_shape_reasons():
    from hstu_amd import unsupported_shape_reason

    bf = torch.zeros(4, 2, 128, dtype=torch.bfloat16)
    assert "GPU" in unsupported_shape_reason(bf, bf, bf)
    assert "head dim" in unsupported_shape_reason(*(torch.zeros(4, 2, 96, dtype=torch.bfloat16),) * 3)
    assert "dtype" in unsupported_shape_reason(*(torch.zeros(4, 2, 128),) * 3)
    assert "d_v" in unsupported_shape_reason(bf, bf, torch.zeros(4, 2, 64, dtype=torch.bfloat16))
    f8 = torch.zeros(4, 2, 64, dtype=torch.float8_e4m3fn)
    assert "e4m3 head dim" in unsupported_shape_reason(f8, f8, f8)
    assert "num_softmax_heads" in unsupported_shape_reason(bf, bf, bf, num_softmax_heads=1)


def test_try_entry_points_decline_without_touching_outputs():
    from hstu_amd import try_hstu_attention_bwd, try_hstu_attention_fwd

    q = torch.zeros(4, 2, 128, dtype=torch.bfloat16)
    offs = torch.tensor([0, 4])
    assert try_hstu_attention_fwd(q=q, k=q, v=q, seq_offsets=offs, num_targets=None, N=4, alpha=0.1,
                                  max_attn_len=0, contextual_seq_len=0) is None
    dq = torch.full_like(q, 3.0)
    assert try_hstu_attention_bwd(dout=q, q=q, k=q, v=q, dq=dq, dk=dq, dv=dq, seq_offsets=offs, num_targets=None,
                                  N=4, alpha=0.1, max_attn_len=0, contextual_seq_len=0) is False
    assert torch.all(dq == 3.0)


def test_kernel_ops_raise_instead_of_falling_back():
    from hstu_amd import triton_hstu_attention_fwd

    q = torch.zeros(4, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError):
        triton_hstu_attention_fwd(4, 0.1, q, q, q, torch.tensor([0, 4]), None, 0, 0, None, False, 0)


@pytest.mark.parametrize("kw", [{}, {"num_targets": torch.tensor([2, 1])}, {"max_attn_len": 3},
                                {"contextual_seq_len": 2}])
def test_pytorch_backend_matches_oracle(kw):
    """kernel=PYTORCH (the reference's default backend) restated with torch ops."""
    from hstu_amd import HammerKernel, hstu_mha

    lengths = [7, 4]
    q, k, v = orc.make_qkv(lengths, 2, 8, 0.6, seed=3, dtype=torch.float64)
    offs = orc.offsets_from_lengths(lengths)
    got = hstu_mha(8, 0.3, q, k, v, offs, kernel=HammerKernel.PYTORCH, **kw)
    want = orc.hstu_mha_dense(8, 0.3, q, k, v, offs, kw.get("num_targets"), kw.get("max_attn_len", 0),
                              kw.get("contextual_seq_len", 0), dtype=torch.float64)
    assert torch.allclose(got, want, atol=1e-12)


def test_pytorch_backend_bias_and_autograd():
    from hstu_amd import HammerKernel, hstu_mha

    lengths = [5, 6]
    q, k, v = orc.make_qkv(lengths, 2, 4, 0.6, seed=4, dtype=torch.float64)
    offs = orc.offsets_from_lengths(lengths)
    bias = orc.make_bias(2, 3, seed=1, std=0.4).double()
    got = hstu_mha(6, 0.5, q, k, v, offs, kernel=HammerKernel.PYTORCH, attn_bias=bias)
    want = orc.hstu_mha_dense(6, 0.5, q, k, v, offs, attn_bias=bias, dtype=torch.float64)
    assert torch.allclose(got, want, atol=1e-12)


def test_hstu_mha_asserts_causal():
    from hstu_amd import hstu_mha

    q = torch.zeros(4, 1, 8)
    with pytest.raises(Exception):
        hstu_mha(4, 0.1, q, q, q, torch.tensor([0, 4]), causal=False)


def test_bench_rejects_multi_gpu():
    r = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stdout
