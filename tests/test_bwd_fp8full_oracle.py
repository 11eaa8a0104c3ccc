"""Pins of the full-FP8 backward oracle (oracle/hstu_bwd_fp8full_oracle.py)
on the CPU: the pre-scale closed forms, the power-of-two normaliser, the
exact backward with the casts off, the e4m3 error bound with them on, and
planted mistakes (a dropped dO group scale, a dropped P pre-scale) that
the bound catches."""

import math

import pytest
import torch

from oracle import hstu_bwd_fp8full_oracle as FO
from oracle import hstu_do_fp8_oracle as DO
from oracle import hstu_oracle as orc


def test_prescales_closed_forms():
    assert FO.prescales(4096) == (2.0 ** 15, 2.0 ** 9)
    assert FO.prescales(1000) == (2.0 ** 13, 2.0 ** 7)
    assert FO.prescales(1024) == (2.0 ** 13, 2.0 ** 7)
    assert FO.prescales(1025) == (2.0 ** 14, 2.0 ** 8)
    assert FO.prescales(2) == (2.0 ** 4, 2.0 ** -2)
    assert FO.prescales(4096, dsc_k=-5) == (2.0 ** 15, 2.0 ** 7)
    assert FO.prescales(2049, 1, -5) == (2.0 ** 13, 2.0 ** 7)


def test_dsc_k_headroom_removes_the_clamp():
    """The production dS pre-scale (K = -5, yambda_5b.gin:3764-3799) quarters
    the default one: on these inputs the default clamps some dS at 448
    (the dO block scale lifts a group's largest row to the top of the e4m3
    range), K = -5 clamps none, and its dk is no farther from the exact
    backward than the clamped one."""
    lengths = [300, 77, 129]
    N = max(lengths)
    q8, k8, v8, sq, sk, sv, offs, dout, y, e8 = _case(lengths, seed=11)
    seen = {}
    real = FO.e4m3_sat

    def count(k):
        def cast(x):
            seen[k] = seen.get(k, 0) + int((x.abs() > FO.E4M3_MAX).sum())
            return real(x)
        return cast

    ref = orc.hstu_mha_bwd_closed_form(N, 0.1, orc.dequantize(q8, sq), orc.dequantize(k8, sk),
                                       orc.dequantize(v8, sv), offs, dout.double())
    got = {}
    for k in (-3, -5):
        FO.e4m3_sat = count(k)
        try:
            got[k] = FO.full_fp8_bwd(N, 0.1, q8, k8, v8, sq, sk, sv, offs, y, e8, dsc_k=k)
        finally:
            FO.e4m3_sat = real
    assert seen[-3] > 0 and seen[-5] == 0, seen
    assert orc.rel_l2(ref[1], got[-5][1]) <= orc.rel_l2(ref[1], got[-3][1]) * 1.05
    # K only moves the cast grid: both stay within the contract's e4m3 error
    for k in (-3, -5):
        assert all(orc.rel_l2(r, g) <= 6e-2 for r, g in zip(ref[:3], got[k][:3]))


@pytest.mark.parametrize("s", [1e-3, 0.0078125, 0.3, 1.0, 5.5])
def test_pow2_norm(s):
    n = FO.pow2_norm(s)
    assert 0.5 <= s * n < 1.0 and math.log2(n) == int(math.log2(n))
    assert FO.pow2_norm(0.0) == 1.0


def _case(lengths, H=2, D=128, seed=0):
    q, k, v = orc.make_qkv(lengths, H, D, 1.0, seed=seed)
    offs = orc.offsets_from_lengths(lengths)
    (q8, sq), (k8, sk), (v8, sv) = (orc.quantize_e4m3_rows(t, dim=-1) for t in (q, k, v))
    dout = torch.randn(q.shape, generator=torch.Generator().manual_seed(seed + 3)).to(torch.bfloat16)
    y, e8 = DO.quantize_do_e4m3_blk(dout, offs, max(lengths))
    return q8, k8, v8, sq, sk, sv, offs, dout, y, e8


def test_exact_when_casts_are_off():
    """quantize=False: the closed-form backward of the dequantized inputs and
    dequantized dO, bias gradient included (to the fp32 rounding of the
    dequantized inputs the closed form is given)."""
    lengths = [130, 7, 64]
    N = max(lengths)
    q8, k8, v8, sq, sk, sv, offs, dout, y, e8 = _case(lengths)
    bias = orc.make_bias(2, 64)
    got = FO.full_fp8_bwd(N, 0.1, q8, k8, v8, sq, sk, sv, offs, y, e8, attn_bias=bias, quantize=False)
    dq_do = DO.dequantize_do_e4m3_blk(y, e8).double()
    ref = orc.hstu_mha_bwd_closed_form(N, 0.1, orc.dequantize(q8, sq), orc.dequantize(k8, sk),
                                       orc.dequantize(v8, sv), offs, dq_do, attn_bias=bias)
    for r, g in zip(ref, got):
        assert orc.rel_l2(r, g) <= 1e-6  # the closed form's inputs are fp32 dequantizations


def test_casts_stay_within_e4m3_error_and_catch_planted_mistakes(monkeypatch):
    """With the casts, within 6e-2 relative L2 of the unquantized backward on
    the unquantized dO; dropping the dO group scale (unit E8 bytes) or the P
    pre-scale (P8 = e4m3(silu / N), which underflows) breaks the bound."""
    lengths = [300, 77, 129]
    N = max(lengths)
    q8, k8, v8, sq, sk, sv, offs, dout, y, e8 = _case(lengths, seed=5)
    bias = orc.make_bias(2, 256)
    ref = orc.hstu_mha_bwd_closed_form(N, 0.1, orc.dequantize(q8, sq), orc.dequantize(k8, sk),
                                       orc.dequantize(v8, sv), offs, dout.double(), attn_bias=bias)
    got = FO.full_fp8_bwd(N, 0.1, q8, k8, v8, sq, sk, sv, offs, y, e8, attn_bias=bias)
    for r, g in zip(ref, got):
        assert orc.rel_l2(r, g) <= 6e-2
    unit = torch.full_like(e8, 127)
    wrong = FO.full_fp8_bwd(N, 0.1, q8, k8, v8, sq, sk, sv, offs, y, unit, attn_bias=bias)
    assert all(orc.rel_l2(r, g) > 0.5 for r, g in zip(ref, wrong))
    monkeypatch.setattr(FO, "prescales", lambda n, *k: (1.0, 2.0 ** (math.ceil(math.log2(n)) - 3)))
    no_ssc = FO.full_fp8_bwd(N, 0.1, q8, k8, v8, sq, sk, sv, offs, y, e8, attn_bias=bias)
    assert orc.rel_l2(ref[2], no_ssc[2]) > 0.2
