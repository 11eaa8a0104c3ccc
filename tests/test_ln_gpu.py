"""GPU parity of the output block (LayerNorm * U * dropout, its Philox mask,
the weighted LayerNorm with e4m3 output, and the fused output projection)
through the HIP C ABI, against the CPU oracle (oracle/hstu_ln_oracle.py).

Bars:
* dropout masks: bit-exact (integer work);
* mean / rstd: rtol 1e-5 against float64 on the same bf16 inputs;
* bf16 outputs and gradients: ``assert_close(rtol=1e-2, atol=1e-2)`` (the
  bf16 tolerance), plus relative L2 <= 4e-3;
* e4m3 outputs: within half an e4m3 step of the exact value (|err| <=
  |ref|/16 + 2^-10, plus 1e-3 relative slack for fp32 arithmetic) and >= 99.5%
  of bytes equal to torch's round-to-nearest-even cast of the float64 value;
* dweight / dbias (fp32, fixed-order sums): rtol 1e-3 against float64.
"""

import numpy as np
import pytest
import torch

import hstu_amd.hstu_linear as L_mod

from oracle import hstu_ln_oracle as L

pytestmark = pytest.mark.gpu

DEV = "cuda"
ACT = {"none": "none", "silu": "silu", "sigmoid": "sigmoid"}


def _ops():
    import hstu_amd

    return hstu_amd


def _inputs(N, D, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(N, D, generator=g) * 1.5 + 0.3).to(torch.bfloat16)
    u = torch.randn(N, D, generator=g).to(torch.bfloat16)
    w = (1.0 + 0.2 * torch.randn(D, generator=g)).to(torch.bfloat16)
    b = (0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    return x, u, w, b


def _rel_l2(ref, got):
    ref, got = ref.double(), got.double()
    return float((got - ref).norm() / ref.norm().clamp_min(1e-30))


def _bf16_close(got, ref, what):
    got = got.float().cpu()
    torch.testing.assert_close(got, ref.float(), rtol=1e-2, atol=1e-2, msg=what)
    assert _rel_l2(ref, got) <= 4e-3, what


def _e4m3_close(got8, ref, inv_scale, what):
    r = (ref.double() * inv_scale).clamp(-448.0, 448.0)
    g = got8.cpu().float().double()
    bound = r.abs() / 16 * (1 + 1e-3) + 2.0 ** -10
    bad = (g - r).abs() > bound
    assert not bad.any(), f"{what}: {int(bad.sum())} elements beyond half an e4m3 step"
    exact = (got8.cpu().view(torch.uint8) == L.e4m3_bytes(ref, inv_scale).view(torch.uint8)).float().mean()
    assert float(exact) >= 0.995, f"{what}: only {float(exact):.4f} of bytes equal"


@pytest.mark.parametrize("mask16", [False, True])
@pytest.mark.parametrize("N,D,nm,p", [(1, 512, 3, 0.3), (13, 256, 2, 0.1), (1000, 512, 3, 0.3),
                                      (77, 512, 1, 0.5), (64, 256, 3, 1.0), (40, 512, 3, 0.0)])
def test_dropout_mask_bitexact(hip_lib, mask16, N, D, nm, p, monkeypatch):
    ops = _ops()
    monkeypatch.setattr(L_mod, "_mask16", bool(mask16))
    seed = (123456789 << 20) + 987  # both key words non-zero
    got = ops.create_dropout_mask(N, D, nm == 3 or nm == 2, nm == 3, p, seed, torch.device(DEV))
    ref = L.dropout_mask(N, D, nm, p, seed, mask16)
    assert np.array_equal(got.cpu().numpy(), ref)


CASES = [
    # act, silu_u, concat_u, concat_x, training, mask16, fp8, D
    ("silu", True, True, True, True, True, True, 512),    # production (yambda_5b.gin, FP8 out)
    ("silu", True, True, True, True, False, False, 512),
    ("none", False, True, True, False, False, False, 512),
    ("sigmoid", False, False, True, True, True, False, 256),
    ("none", False, True, False, True, False, True, 256),
    ("silu", False, False, False, True, True, False, 512),
    ("none", False, False, False, False, False, False, 256),
]


def _oracle_fwd(x, u, w, b, eps, p, mask, act, silu_u, cu, cx):
    return L.ln_mul_dropout_fwd(x.double(), u.double(), w.double(), b.double(), eps, dropout_ratio=p, mask=mask,
                                silu_u=silu_u, concat_u=cu, concat_x=cx, mul_u_activation_type=act)


@pytest.mark.parametrize("act,silu_u,cu,cx,training,mask16,fp8,D", CASES)
def test_ln_mul_dropout_fwd(hip_lib, monkeypatch, act, silu_u, cu, cx, training, mask16, fp8, D):
    ops = _ops()
    monkeypatch.setattr(L_mod, "_mask16", bool(mask16))
    N, p, eps, seed, inv = 1003, 0.3, 1e-6, 2 ** 40 + 17, 8.0
    x, u, w, b = _inputs(N, D, seed=1)
    y, mean, rstd, bd, nw, s, mask = ops.triton_layer_norm_mul_dropout_fwd(
        x.to(DEV), u.to(DEV), w.to(DEV), b.to(DEV), eps, p, training, silu_u, cu, cx, act, seed,
        output_fp8=fp8, inv_scale=inv)
    assert bd == D and s == seed
    ref_mask = L.dropout_mask(N, D, 1 + cu + cx, p, seed, mask16) if training else None
    if training:
        assert np.array_equal(mask.cpu().numpy(), ref_mask)
    else:
        assert mask is None
    ry, rmean, rrstd = _oracle_fwd(x, u, w, b, eps, p, ref_mask, act, silu_u, cu, cx)
    torch.testing.assert_close(mean.cpu().double(), rmean, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(rstd.cpu().double(), rrstd, rtol=1e-5, atol=1e-6)
    assert y.shape == ry.shape
    if fp8:
        _e4m3_close(y, ry, inv, "y e4m3")
    else:
        _bf16_close(y, ry, "y")
        if cx and not training:  # the x block is a verbatim copy
            off = D if cu else 0
            assert torch.equal(y[:, off:off + D].cpu(), x)


@pytest.mark.parametrize("act,silu_u,cu,cx,training,mask16,fp8,D", CASES)
def test_ln_mul_dropout_bwd(hip_lib, monkeypatch, act, silu_u, cu, cx, training, mask16, fp8, D):
    ops = _ops()
    monkeypatch.setattr(L_mod, "_mask16", bool(mask16))
    N, p, eps, seed = 2051, 0.3, 1e-6, 99
    x, u, w, b = _inputs(N, D, seed=2)
    xd, ud, wd, bd_ = (t.to(DEV) for t in (x, u, w, b))
    y, mean, rstd, BD, nw, s, mask = ops.triton_layer_norm_mul_dropout_fwd(
        xd, ud, wd, bd_, eps, p, training, silu_u, cu, cx, act, seed)
    dy = torch.randn(y.shape, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    dx, du, dw, db, yre = ops.triton_layer_norm_mul_dropout_bwd(
        dy.to(DEV), xd, ud, wd, bd_, mean, rstd, BD, nw, eps, training, p, s, silu_u, cu, cx, act,
        compute_y=True, random_mask=mask)
    ref_mask = L.dropout_mask(N, D, 1 + cu + cx, p, seed, mask16) if training else None
    rdx, rdu, rdw, rdb = L.ln_mul_dropout_bwd(dy.double(), x.double(), u.double(), w.double(), b.double(), eps,
                                              dropout_ratio=p, mask=ref_mask, silu_u=silu_u, concat_u=cu,
                                              concat_x=cx, mul_u_activation_type=act)
    _bf16_close(dx, rdx, "dx")
    _bf16_close(du, rdu, "du")
    assert dw.dtype == w.dtype and db.dtype == b.dtype
    for name, got, ref in (("dweight", dw, rdw), ("dbias", db, rdb)):
        got = got.float().cpu().double()
        # bf16 result of an fp32 sum: one bf16 rounding (2^-8) on top of 1e-3
        torch.testing.assert_close(got, ref, rtol=5e-3, atol=1e-3 * float(ref.abs().max()), msg=name)
    # the recomputed y is the forward's y (same fp32 arithmetic, same mask)
    diff = (yre.float() - y.float()).abs()
    assert float((diff <= 2.0 ** -7 * y.float().abs()).float().mean()) == 1.0
    # training backward without the saved mask redraws it from the seed
    if training:
        dx2, du2, _, _, _ = ops.triton_layer_norm_mul_dropout_bwd(
            dy.to(DEV), xd, ud, wd, bd_, mean, rstd, BD, nw, eps, training, p, s, silu_u, cu, cx, act)
        assert torch.equal(dx2, dx) and torch.equal(du2, du)


def test_bwd_deterministic_and_du_row_width(hip_lib):
    ops = _ops()
    N, D = 3001, 512
    x, u, w, b = (t.to(DEV) for t in _inputs(N, D, seed=4))
    y, mean, rstd, BD, nw, s, mask = ops.triton_layer_norm_mul_dropout_fwd(
        x, u, w, b, 1e-6, 0.3, True, True, True, True, "silu", 5)
    dy = torch.randn(y.shape, device=DEV).to(torch.bfloat16)
    r1 = ops.triton_layer_norm_mul_dropout_bwd(dy, x, u, w, b, mean, rstd, BD, nw, 1e-6, True, 0.3, s, True,
                                               True, True, "silu", random_mask=mask)
    r2 = ops.triton_layer_norm_mul_dropout_bwd(dy, x, u, w, b, mean, rstd, BD, nw, 1e-6, True, 0.3, s, True,
                                               True, True, "silu", random_mask=mask, du_row_width=2048)
    for a, c in zip(r1[:4], r2[:4]):
        assert torch.equal(a, c)
    assert r2[1].stride(0) == 2048


@pytest.mark.parametrize("D,fp8", [(512, True), (512, False), (256, True)])
def test_weighted_layer_norm(hip_lib, D, fp8):
    ops = _ops()
    N, eps, inv = 777, 1e-5, 1.0 / 0.02
    x, _, w, b = _inputs(N, D, seed=6)
    y, mean, rstd = ops.triton_weighted_layer_norm_fwd(x.to(DEV), w.to(DEV), b.to(DEV), eps, output_fp8=fp8,
                                                       inv_scale=inv)
    ry, rmean, rrstd = L.ln_mul_dropout_fwd(x.double(), None, w.double(), b.double(), eps)
    torch.testing.assert_close(rstd.cpu().double(), rrstd, rtol=1e-5, atol=1e-6)
    if fp8:
        _e4m3_close(y, ry, inv, "LN e4m3")
    else:
        _bf16_close(y, ry, "LN")
    dy = torch.randn(N, D, generator=torch.Generator().manual_seed(8)).to(torch.bfloat16)
    dx, dw, db = ops.triton_weighted_layer_norm_bwd(dy.to(DEV), x.to(DEV), w.to(DEV), b.to(DEV), mean, rstd, True,
                                                    eps, D)
    rdx, _, rdw, rdb = L.ln_mul_dropout_bwd(dy.double(), x.double(), None, w.double(), b.double(), eps)
    _bf16_close(dx, rdx, "LN dx")
    torch.testing.assert_close(dw.float().cpu().double(), rdw, rtol=5e-3, atol=1e-3 * float(rdw.abs().max()))
    torch.testing.assert_close(db.float().cpu().double(), rdb, rtol=5e-3, atol=1e-3 * float(rdb.abs().max()))


@pytest.mark.parametrize("fp8", [False, True])
def test_hstu_compute_output_fwd_bwd(hip_lib, monkeypatch, fp8):
    """The output block with the production flags (modules/stu.py:621-651):
    concat_u = concat_x = True, silu, dropout 0.3 in training, y recomputed in
    the backward; FP8 e4m3 LN output into the FP8 projection when a scale is
    given."""
    from oracle import hstu_oracle as orc

    ops = _ops()
    monkeypatch.setattr(L_mod, "_mask16", True)
    N, D, Dout, p, eps, seed, sc = 1500, 512, 512, 0.3, 1e-6, 4242, 0.05
    attn, u, nw, nb = _inputs(N, D, seed=9)
    g = torch.Generator().manual_seed(10)
    x = torch.randn(N, Dout, generator=g).to(torch.bfloat16)
    W = (torch.randn(3 * D, Dout, generator=g) * 0.03).to(torch.bfloat16)
    leaves = [t.to(DEV).requires_grad_(True) for t in (attn, u, x, nw, nb, W)]
    out = ops.triton_hstu_compute_output(leaves[0], leaves[1], leaves[2], leaves[3], leaves[4], leaves[5], eps, p,
                                         True, True, True, True, "silu", seed=seed, recompute_y_in_backward=True,
                                         fp8_output_scale=torch.full((1, 1), sc, device=DEV) if fp8 else None)
    dout = torch.randn(N, Dout, generator=g).to(torch.bfloat16)
    out.backward(dout.to(DEV))
    mask = L.dropout_mask(N, D, 3, p, seed, True)
    args = [t.double().requires_grad_(True) for t in (attn, u, x, nw, nb, W)]
    y, _, _ = L.ln_mul_dropout_fwd(args[0], args[1], args[3], args[4], eps, dropout_ratio=p, mask=mask, silu_u=True,
                                   concat_u=True, concat_x=True, mul_u_activation_type="silu")
    ref = args[2] + y @ args[5]
    ref.backward(dout.double())
    got = out.detach().float().cpu().double()
    if fp8:  # the GEMM consumes e4m3(y / scale) and per-column e4m3 weights
        y_q = L.e4m3_bytes(y.detach(), 1.0 / sc).double() * sc
        w8, ws = orc.quantize_e4m3_rows(W.t().contiguous().float())
        w_q = orc.dequantize(w8, ws).double().t()
        ref_out = x.double() + y_q @ w_q
        assert _rel_l2(ref_out, got) <= 1e-2, _rel_l2(ref_out, got)
    else:
        _bf16_close(got, ref.detach(), "out")
    for name, leaf, a in zip(("dattn", "du", "dx", "dnorm_w", "dnorm_b", "dW"), leaves, args):
        g_ = leaf.grad.float().cpu().double()
        assert _rel_l2(a.grad, g_) <= 1e-2, (name, _rel_l2(a.grad, g_))


def test_hstu_compute_output_dispatch(hip_lib):
    """``hstu_compute_output`` routes TRITON / HIP to the HIP kernels: eval
    mode (no dropout) matches the PYTORCH backend to the bf16 bar."""
    ops = _ops()
    N, D = 300, 512
    attn, u, nw, nb = (t.to(DEV) for t in _inputs(N, D, seed=11))
    x = torch.randn(N, D, device=DEV).to(torch.bfloat16)
    W = (torch.randn(3 * D, D, device=DEV) * 0.03).to(torch.bfloat16)
    kw = dict(norm_eps=1e-6, output_weight=W, num_heads=4, linear_dim=128, dropout_ratio=0.3, training=False,
              concat_u=True, concat_x=True, mul_u_activation_type="silu", group_norm=False,
              recompute_y_in_backward=True)
    a = ops.hstu_compute_output(attn, u, x, nw, nb, kernel=ops.HammerKernel.TRITON, **kw)
    b = ops.hstu_compute_output(attn, u, x, nw, nb, kernel=ops.HammerKernel.PYTORCH, **kw)
    torch.testing.assert_close(a.float(), b.float(), rtol=1e-2, atol=2e-2)


def test_ln_bwd_residual_gradient(hip_lib):
    """A residual branch's gradient of x folded into the plain LayerNorm's
    backward (``dres``, as the layer passes the output block's): dx =
    the LN backward + dres with one rounding, against float64 at the bf16 bar;
    dweight / dbias unchanged bit for bit."""
    N, D, eps = 1031, 512, 1e-6
    x, _, w, b = _inputs(N, D, seed=8)
    g = torch.Generator().manual_seed(9)
    dxn = torch.randn(N, D, generator=g).to(torch.bfloat16)
    dres = (4.0 * torch.randn(N, D, generator=g)).to(torch.bfloat16)
    xd, wd, bd = (t.to(DEV) for t in (x, w, b))
    _, mean, rstd, _ = L_mod._ln_fwd(xd, None, wd, bd, eps, 0.0, False, False, False, False, "none", 0, False, 1.0)
    args = (dxn.to(DEV), xd, None, wd, bd, mean, rstd, 0.0, None, False, False, False, "none", False)
    dx0, _, dw0, db0, _ = L_mod._ln_bwd(*args)
    dx, _, dw, db, _ = L_mod._ln_bwd(*args, dres=dres.to(DEV))
    rdx, _, _, _ = L.ln_mul_dropout_bwd(dxn.double(), x.double(), None, w.double(), b.double(), eps)
    _bf16_close(dx, rdx + dres.double(), "dx with the residual gradient")
    assert torch.equal(dw, dw0) and torch.equal(db, db0)
    # dx rounds the fp32 sum once, dx0 was rounded before the sum: each within
    # half a bf16 step (2^-8 relative) of its exact value
    d = (dx.float() - (dx0.float() + dres.to(DEV).float())).abs()
    assert float((d <= 2.0 ** -7 * (dx.float().abs() + dx0.float().abs()) + 1e-6).float().mean()) == 1.0


def test_ln_params_bf16_and_fp32_agree(hip_lib):
    """The LayerNorm kernels read bf16 parameters as they are (param_dtype
    bf16) and fp32 ones as fp32: the same values give bitwise-equal outputs
    and gradients (the parameter gradients come back in each parameter's
    dtype, so they are compared in the first call's), and a mix of the two
    goes as fp32."""
    ops = _ops()
    N, D = 1001, 512
    x, u, w, b = (t.to(DEV) for t in _inputs(N, D, seed=6))
    outs = []
    for ww, bb in ((w, b), (w.float(), b.float()), (w, b.float())):
        y, mean, rstd, BD, nw, s, mask = ops.triton_layer_norm_mul_dropout_fwd(
            x, u, ww, bb, 1e-6, 0.3, True, True, True, True, "silu", 5)
        dy = torch.randn(y.shape, device=DEV, generator=torch.Generator(device=DEV).manual_seed(3)).to(torch.bfloat16)
        r = ops.triton_layer_norm_mul_dropout_bwd(dy, x, u, ww, bb, mean, rstd, BD, nw, 1e-6, True, 0.3, s, True,
                                                  True, True, "silu", random_mask=mask)
        outs.append((y, mean, rstd) + tuple(r[:4]))
    for other in outs[1:]:
        for a, c in zip(outs[0], other):
            assert torch.equal(a, c.to(a.dtype))
