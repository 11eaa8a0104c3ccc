"""Pins of the FP8 P.V forward oracle (oracle/hstu_fwd_pv8_oracle.py) on the
CPU: with the cast off it equals the pinned float64 attention; the V-scale
group exponents against a brute-force loop; with the cast on, the e4m3 error
bound, and a planted mistake (P cast to e5m2) that the bound catches.  Also the product's reading of DLRM_HSTU_FP8_FWD_PV_SCALE against the
reference's documented rules (hstu_flydsl_mha.py:2224-2264)."""

import math

import pytest
import torch

from oracle import hstu_fwd_pv8_oracle as PV
from oracle import hstu_oracle as orc


def _case(lengths, H=2, D=128, seed=0, per_tensor=False, std=1.0):
    q, k, v = orc.make_qkv(lengths, H, D, std, seed=seed)
    offs = orc.offsets_from_lengths(lengths)
    if per_tensor:
        outs = []
        for t in (q, k, v):
            q8, s = orc.quantize_e4m3_per_tensor(t)
            outs.append((q8, s.reshape(1)))
    else:
        outs = [orc.quantize_e4m3_rows(t, dim=-1) for t in (q, k, v)]
    (q8, sq), (k8, sk), (v8, sv) = outs
    return q8, k8, v8, sq, sk, sv, offs


def _deq(x8, s):
    """float64 dequantization (per-tensor scalar or [T, H] scales)."""
    return x8.double() * (float(s) if s.numel() == 1 else s.double().unsqueeze(-1))


@pytest.mark.parametrize("per_tensor", [False, True])
@pytest.mark.parametrize("with_bias", [False, True])
def test_exact_without_the_cast(per_tensor, with_bias):
    lengths = [130, 7, 64, 1, 200]
    N = 256
    q8, k8, v8, sq, sk, sv, offs = _case(lengths, per_tensor=per_tensor, seed=3)
    bias = orc.make_bias(2, 128) if with_bias else None
    got = PV.fwd_pv8(N, 0.1, q8, k8, v8, sq, sk, sv, offs, attn_bias=bias, quantize=False)
    want = orc.hstu_mha_dense(N, 0.1, _deq(q8, sq), _deq(k8, sk), _deq(v8, sv), offs, attn_bias=bias,
                              dtype=torch.float64)
    assert orc.rel_l2(want, got) <= 1e-12


def test_group_exponents_brute_force():
    g = torch.Generator().manual_seed(5)
    L = 150
    sv = torch.rand(L, generator=g, dtype=torch.float64) * 0.05
    sv[70:75] = 0.0
    E = PV.group_exponents(sv, L)
    for k in range(L):
        t0 = 64 * (k // 64)
        grp = [j for j in range(t0, min(t0 + 64, L)) if (j - t0) // 16 % 2 == (k - t0) // 16 % 2]
        assert E[k] == math.frexp(max(float(sv[j]) for j in grp))[1]
    r = sv * torch.exp2(-E)
    for t0 in range(0, L, 64):
        for gsel in (0, 1):
            idx = [j for j in range(t0, min(t0 + 64, L)) if (j - t0) // 16 % 2 == gsel]
            assert 0.5 <= float(r[idx].max()) < 1.0
    assert torch.all(PV.group_exponents(torch.zeros(40, dtype=torch.float64), 40) == 0)


@pytest.mark.parametrize("per_tensor", [False, True])
def test_cast_error_bound_and_planted_mistake(per_tensor, monkeypatch):
    """With the cast the output stays within 3.5e-2 relative L2 of the
    unquantized forward (2.6 % measured: e4m3 keeps 3 mantissa bits of P), and
    the cast is really there (> 1e-3).  A planted mistake, P cast to e5m2 (2
    mantissa bits), doubles the error and breaks the bound."""
    lengths = [300, 77, 129, 512]
    N = 600
    q8, k8, v8, sq, sk, sv, offs = _case(lengths, per_tensor=per_tensor, seed=7)
    bias = orc.make_bias(2, 256)
    exact = PV.fwd_pv8(N, 0.1, q8, k8, v8, sq, sk, sv, offs, attn_bias=bias, quantize=False)
    got = PV.fwd_pv8(N, 0.1, q8, k8, v8, sq, sk, sv, offs, attn_bias=bias)
    e = orc.rel_l2(exact, got)
    assert 1e-3 < e <= 3.5e-2, e
    monkeypatch.setattr(PV, "e4m3_sat",
                        lambda x: x.clamp(-57344.0, 57344.0).to(torch.float8_e5m2).to(torch.float64))
    wrong = PV.fwd_pv8(N, 0.1, q8, k8, v8, sq, sk, sv, offs, attn_bias=bias)
    assert orc.rel_l2(exact, wrong) > 3.5e-2


@pytest.mark.parametrize("raw,want", [(None, 10.04), ("", 10.04), ("pow2", 8.0), ("POW2", 8.0), ("0", 8.0),
                                      ("16", 16.0), ("4", 4.0), ("32", 32.0), ("12.3456789", 12.345679)])
def test_pv_scale_parsing(raw, want, monkeypatch):
    from hstu_amd import hstu_attention as A

    if raw is None:
        monkeypatch.delenv("DLRM_HSTU_FP8_FWD_PV_SCALE", raising=False)
    else:
        monkeypatch.setenv("DLRM_HSTU_FP8_FWD_PV_SCALE", raw)
    assert A.fp8_fwd_pv_scale() == want


@pytest.mark.parametrize("raw", ["3.99", "33", "nan", "inf", "abc", "-8"])
def test_pv_scale_parsing_rejects(raw, monkeypatch):
    from hstu_amd import hstu_attention as A

    monkeypatch.setenv("DLRM_HSTU_FP8_FWD_PV_SCALE", raw)
    with pytest.raises(ValueError):
        A.fp8_fwd_pv_scale()


@pytest.mark.parametrize("raw,want", [(None, False), ("0", False), ("1", True), ("true", False), ("", False)])
def test_pv_switch(raw, want, monkeypatch):
    from hstu_amd import hstu_attention as A

    if raw is None:
        monkeypatch.delenv("DLRM_HSTU_FP8_FWD_PV", raising=False)
    else:
        monkeypatch.setenv("DLRM_HSTU_FP8_FWD_PV", raw)
    assert A.fp8_fwd_pv_enabled() is want
