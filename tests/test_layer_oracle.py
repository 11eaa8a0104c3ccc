"""Pins of the layer oracle's production attention step
(``hstu_layer_oracle.production_attention``: the FP8 P.V forward and the
full-FP8 backward on the block-quantized bf16 dO) on the CPU.

* casts off: equal to the float64 dense attention and its autograd
  gradients (dq, dk, dv, dbias) to 1e-9 -- this pins the wiring (the codes
  recovered from the dequantized inputs, the scales, the argument order);
* casts on: within the contract's e4m3 error of the exact attention
  (output 3.5e-2, gradients 6e-2 relative L2), and a planted mistake (a dS
  pre-scale that saturates, or q and k swapped) breaks that bound;
* the whole layer with the production attention stays within the same error
  of the layer with the dense attention.
"""

import numpy as np
import pytest
import torch

from oracle import hstu_layer_oracle as LO
from oracle import hstu_oracle as orc


def _inputs(lengths, H=2, D=128, s=0.02, seed=0):
    g = torch.Generator().manual_seed(seed)
    T = int(sum(lengths))
    codes = [(torch.randn(T, H, D, generator=g) * 60).clamp(-448, 448).to(torch.float8_e4m3fn).double()
             for _ in range(3)]
    bias = orc.make_bias(H, 128, seed=seed + 1, std=0.3).double()
    dout = torch.randn(T, H, D, generator=g, dtype=torch.float64)
    return [c * s for c in codes], bias, dout


def _grads(fn, q, k, v, bias, dout):
    leaves = [t.clone().requires_grad_(True) for t in (q, k, v, bias)]
    out = fn(*leaves)
    out.backward(dout)
    return out.detach(), [t.grad for t in leaves]


def test_production_attention_exact_without_casts():
    lengths = [130, 7, 64, 1]
    N, alpha, s = 130, 0.1, 0.02
    (q, k, v), bias, dout = _inputs(lengths, s=s)
    offs = orc.offsets_from_lengths(lengths)
    got, gg = _grads(lambda a, b, c, d: LO.production_attention(a, b, c, s, offs, N, alpha, attn_bias=d,
                                                                quantize=False), q, k, v, bias, dout)
    ref, rg = _grads(lambda a, b, c, d: orc.hstu_mha_dense(N, alpha, a, b, c, offs, attn_bias=d,
                                                           dtype=torch.float64), q, k, v, bias, dout)
    assert orc.rel_l2(ref, got) <= 1e-9
    for name, r, g in zip(("dq", "dk", "dv", "dbias"), rg, gg):
        assert orc.rel_l2(r, g) <= 1e-9, name


def test_production_attention_casts_within_contract_error(monkeypatch):
    lengths = [300, 77, 129]
    N, alpha, s = 300, 1.0 / 128 ** 0.5, 0.02
    (q, k, v), bias, dout = _inputs(lengths, s=s, seed=3)
    offs = orc.offsets_from_lengths(lengths)
    ref, rg = _grads(lambda a, b, c, d: orc.hstu_mha_dense(N, alpha, a, b, c, offs, attn_bias=d,
                                                           dtype=torch.float64), q, k, v, bias, dout)

    def run(dsc_k=-5):
        return _grads(lambda a, b, c, d: LO.production_attention(a, b, c, s, offs, N, alpha, attn_bias=d,
                                                                 dsc_k=dsc_k), q, k, v, bias, dout)

    got, gg = run()
    assert orc.rel_l2(ref, got) <= 3.5e-2
    for name, r, g in zip(("dq", "dk", "dv"), rg, gg):
        assert orc.rel_l2(r, g) <= 6e-2, name
    # planted: a dS pre-scale 2^11 too large, so most dS saturate at 448
    _, bg = run(dsc_k=6)
    assert orc.rel_l2(rg[0], bg[0]) > 0.2 and orc.rel_l2(rg[1], bg[1]) > 0.2
    # planted: q and k swapped inside the step
    swapped, sg = _grads(lambda a, b, c, d: LO.production_attention(b, a, c, s, offs, N, alpha, attn_bias=d,
                                                                    dsc_k=-5), q, k, v, bias, dout)
    assert orc.rel_l2(ref, swapped) > 0.2


def test_layer_with_production_attention_near_dense():
    """hstu_layer_ref(attention="production") against the dense-attention
    layer at the same activation scales: output within 2e-2, every gradient
    within 8e-2 (the attention's e4m3 P / dS / dO casts on top of the
    layer's own quantizers)."""
    lengths = np.array([200, 33, 64])
    T, N = int(lengths.sum()), 200
    g = torch.Generator().manual_seed(9)
    x = torch.randn(T, 512, generator=g).to(torch.bfloat16)
    dy = torch.randn(T, 512, generator=g).double()
    params = LO.make_layer_params(512, seed=2)
    bias = orc.make_bias(4, 256, seed=4)
    res = {}
    for att in ("dense", "production"):
        xr = x.double().requires_grad_(True)
        pr = {k: v.double().requires_grad_(True) for k, v in params.items()}
        br = bias.double().requires_grad_(True)
        out = LO.hstu_layer_ref(xr, pr, lengths, N, s_x=0.02, s_qkv=0.01, s_out=0.05, attn_bias=br,
                                attention=att, dsc_k=-5)
        out.backward(dy)
        res[att] = (out.detach(), xr.grad, br.grad, {k: t.grad for k, t in pr.items()})
    d, p = res["dense"], res["production"]
    assert orc.rel_l2(d[0], p[0]) <= 2e-2
    assert orc.rel_l2(d[1], p[1]) <= 8e-2 and orc.rel_l2(d[2], p[2]) <= 8e-2
    for k in params:
        assert orc.rel_l2(d[3][k], p[3][k]) <= 8e-2, k
    with pytest.raises(ValueError):
        LO.hstu_layer_ref(x.double(), {k: v.double() for k, v in params.items()}, lengths, N, s_x=0.02,
                          s_qkv=None, attention="production")
