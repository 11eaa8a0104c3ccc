"""GPU parity of one whole HSTU layer (BASELINE config 5's dataflow) through
the HIP kernels, against the float64 layer oracle (oracle/hstu_layer_oracle.py)
on identical seeded inputs, forward and backward.

FP8 layer: the oracle applies the same quantizers (LN output at s_x,
per-column e4m3 weights, V/Q/K at s_qkv, the LN * U output at s_out), so the
remaining differences are bf16 / fp32 rounding and the odd e4m3 rounding flip:
relative L2 <= 1.5e-2 for the output and <= 3e-2 for every gradient.  bf16
layer (no quantizers): output relative L2 <= 1e-2, gradients <= 2e-2.
"""

import numpy as np
import pytest
import torch

import hstu_amd.hstu_linear as L_mod

from oracle import hstu_layer_oracle as LO
from oracle import hstu_ln_oracle as L
from oracle import hstu_oracle as orc

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rel_l2(ref, got):
    ref, got = ref.double(), got.double()
    return float((got - ref).norm() / ref.norm().clamp_min(1e-30))


def _calibrate(x, params):
    """amax * 1.25 / 448 of each quantized activation, from a float64 pass."""
    p = {k: v.double() for k, v in params.items()}
    xn = torch.nn.functional.layer_norm(x.double(), (x.shape[1],), p["input_norm_weight"], p["input_norm_bias"],
                                        1e-6)
    vqk = (xn @ p["uvqk_weight"] + p["uvqk_bias"])[:, 512:]
    s_x = float(xn.abs().max()) * 1.25 / 448
    s_qkv = float(vqk.abs().max()) * 1.25 / 448
    return s_x, s_qkv


@pytest.mark.parametrize("fp8,with_bias,dropout", [(True, True, 0.3), (True, False, 0.0), (False, True, 0.3)])
def test_hstu_layer_fwd_bwd(hip_lib, monkeypatch, fp8, with_bias, dropout):
    import hstu_amd

    monkeypatch.setattr(L_mod, "_mask16", True)
    lengths = np.array([300, 77, 512, 129])
    T, N, E, seed = int(lengths.sum()), 512, 512, 77
    g = torch.Generator().manual_seed(3)
    x = torch.randn(T, E, generator=g).to(torch.bfloat16)
    params = LO.make_layer_params(E, seed=4)
    bias = orc.make_bias(4, 1024) if with_bias else None
    s_x, s_qkv = _calibrate(x, params) if fp8 else (None, None)
    s_out = 0.05 if fp8 else None
    dy = torch.randn(T, E, generator=g).to(torch.bfloat16)

    offs = orc.offsets_from_lengths(lengths).to(DEV)
    xd = x.to(DEV).requires_grad_(True)
    pd = {k: v.to(DEV).requires_grad_(True) for k, v in params.items()}
    bd = None if bias is None else bias.to(DEV).requires_grad_(True)
    sc = (lambda s: None if s is None else torch.full((1, 1), s, device=DEV))
    out = hstu_amd.hstu_layer(xd, offs, N, pd, dropout_ratio=dropout, training=True, fp8_input_scale=sc(s_x),
                              fp8_qkv_scale=sc(s_qkv), fp8_output_scale=sc(s_out), attn_bias=bd, seed=seed)
    out.backward(dy.to(DEV))

    mask = L.dropout_mask(T, 512, 3, dropout, seed, True) if dropout > 0 else None
    xr = x.double().requires_grad_(True)
    pr = {k: v.double().requires_grad_(True) for k, v in params.items()}
    br = None if bias is None else bias.double().requires_grad_(True)
    ref = LO.hstu_layer_ref(xr, pr, lengths, N, s_x=s_x, s_qkv=s_qkv, s_out=s_out, dropout_ratio=dropout,
                            mask=mask, attn_bias=br, quantize=fp8)
    ref.backward(dy.double())
    tol_out, tol_grad = (1.5e-2, 3e-2) if fp8 else (1e-2, 2e-2)
    e = _rel_l2(ref.detach(), out.detach().cpu())
    assert e <= tol_out, f"out rel L2 {e:.3e}"
    grads = [("dx", xr.grad, xd.grad)] + [(f"d{k}", pr[k].grad, pd[k].grad) for k in params]
    if bias is not None:
        grads.append(("dbias", br.grad, bd.grad))
    for name, r, got in grads:
        e = _rel_l2(r, got.float().cpu())
        assert e <= tol_grad, f"{name} rel L2 {e:.3e}"


@pytest.mark.parametrize("uvqk_wgrad", ["bf16", "fp8t"])
def test_hstu_layer_fp8_backward_arms(hip_lib, monkeypatch, uvqk_wgrad):
    """The FP8 layer with both e5m2 dgrad arms engaged (output projection and
    UVQK, one warm-up call each): the second step against the oracle with the
    same gradient quantizers at the scales the sites published, at the FP8
    layer's tolerances (output 1.5e-2, gradients 3e-2)."""
    import hstu_amd
    import hstu_amd.bwd_fp8 as B

    monkeypatch.setattr(L_mod, "_mask16", True)
    cfg = B.Fp8BackwardConfig(enabled=True, uvqk=True, warmup_calls=1, uvqk_wgrad_fp8t=uvqk_wgrad == "fp8t",
                              out_wgrad_fp8=uvqk_wgrad == "fp8t")
    B.reset_sites()
    lengths = np.array([300, 77, 512, 129])
    T, N, E = int(lengths.sum()), 512, 512
    g = torch.Generator().manual_seed(13)
    x = torch.randn(T, E, generator=g).to(torch.bfloat16)
    params = LO.make_layer_params(E, seed=5)
    s_x, s_qkv = _calibrate(x, params)
    s_out = 0.05
    dy = torch.randn(T, E, generator=g).to(torch.bfloat16)
    offs = orc.offsets_from_lengths(lengths).to(DEV)
    pd = {k: v.to(DEV).requires_grad_(True) for k, v in params.items()}
    sc = (lambda s: torch.full((1, 1), s, device=DEV))
    for _ in range(2):                      # step 1 publishes the scales (bf16), step 2 runs FP8
        for t in pd.values():
            t.grad = None
        xd = x.to(DEV).requires_grad_(True)
        out = hstu_amd.hstu_layer(xd, offs, N, pd, dropout_ratio=0.0, training=True, fp8_input_scale=sc(s_x),
                                  fp8_qkv_scale=sc(s_qkv), fp8_output_scale=sc(s_out), fp8_backward=cfg)
        out.backward(dy.to(DEV))
    sites = {s: B.find_site(s, layer=0) for s in ("output_projection", "uvqk_projection")}
    assert all(st.calls == 2 for st in sites.values())
    xr = x.double().requires_grad_(True)
    pr = {k: v.double().requires_grad_(True) for k, v in params.items()}
    scales = {s: float(st.scale) for s, st in sites.items()}
    ref = LO.hstu_layer_ref(xr, pr, lengths, N, s_x=s_x, s_qkv=s_qkv, s_out=s_out, dropout_ratio=0.0, quantize=True,
                            grad_scales=scales, fp8_wgrad=("uvqk_projection", "output_projection") if uvqk_wgrad == "fp8t" else ())
    ref.backward(dy.double())
    e = _rel_l2(ref.detach(), out.detach().cpu())
    assert e <= 1.5e-2, f"out rel L2 {e:.3e}"
    for name, r, got in [("dx", xr.grad, xd.grad)] + [(f"d{k}", pr[k].grad, pd[k].grad) for k in params]:
        e = _rel_l2(r, got.float().cpu())
        assert e <= 3e-2, f"{name} rel L2 {e:.3e}"
    B.reset_sites()


def test_hstu_layer_calibrated_scale_states_no_host_sync(hip_lib, monkeypatch):
    """The layer with the reference's per-layer scale state buffers
    ([2 + steps] fp32, all zero): the first CALIBRATION_STEPS calls run bf16
    and fill the amax histories; then the scales freeze at max(history) *
    1.5 / 448 (their closed form, from the recorded histories), the layer
    runs FP8, and a whole fwd + bwd step makes no host synchronisation
    (torch.cuda.set_sync_debug_mode("error")).  The FP8 step matches the
    float64 layer oracle at the frozen scales (output 1.5e-2, gradients 3e-2)."""
    import hstu_amd
    from hstu_amd import fp8 as F

    monkeypatch.setattr(L_mod, "_mask16", True)
    lengths = np.array([300, 77, 512, 129])
    T, N, E = int(lengths.sum()), 512, 512
    g = torch.Generator().manual_seed(23)
    x = torch.randn(T, E, generator=g).to(torch.bfloat16)
    params = LO.make_layer_params(E, seed=6)
    dy = torch.randn(T, E, generator=g).to(torch.bfloat16)
    offs = orc.offsets_from_lengths(lengths).to(DEV)
    pd = {k: v.to(DEV).requires_grad_(True) for k, v in params.items()}
    states = {n: torch.zeros(F.fp8_scale_state_size(), device=DEV) for n in ("in", "qkv", "out")}
    x_dev, dy_dev = x.to(DEV), dy.to(DEV)   # inputs resident on the device before the checked step

    def step():
        for t in pd.values():
            t.grad = None
        xd = x_dev.detach().requires_grad_(True)
        out = hstu_amd.hstu_layer(xd, offs, N, pd, dropout_ratio=0.0, training=True,
                                  fp8_input_scale=states["in"], fp8_qkv_scale=states["qkv"],
                                  fp8_output_scale=states["out"], fp8_backward=hstu_amd.bwd_fp8.Fp8BackwardConfig())
        out.backward(dy_dev)
        return xd, out

    for _ in range(F.CALIBRATION_STEPS):
        assert not F.scale_ready(states["in"])
        step()
    for n, st in states.items():
        hist = st[2:].cpu()
        assert F.scale_ready(st) and float(st[1]) == F.CALIBRATION_STEPS and bool((hist > 0).all()), n
        assert float(st[0]) == pytest.approx(float(hist.max()) * 1.5 / 448, rel=1e-6), n
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        xd, out = step()
    finally:
        torch.cuda.set_sync_debug_mode("default")
    s_x, s_qkv, s_out = (float(states[n][0]) for n in ("in", "qkv", "out"))
    xr = x.double().requires_grad_(True)
    pr = {k: v.double().requires_grad_(True) for k, v in params.items()}
    ref = LO.hstu_layer_ref(xr, pr, lengths, N, s_x=s_x, s_qkv=s_qkv, s_out=s_out, dropout_ratio=0.0, quantize=True)
    ref.backward(dy.double())
    e = _rel_l2(ref.detach(), out.detach().cpu())
    assert e <= 1.5e-2, f"out rel L2 {e:.3e}"
    for name, r, got in [("dx", xr.grad, xd.grad)] + [(f"d{k}", pr[k].grad, pd[k].grad) for k in params]:
        e = _rel_l2(r, got.float().cpu())
        assert e <= 3e-2, f"{name} rel L2 {e:.3e}"


def test_hstu_layer_fused_outproj_backward(hip_lib, monkeypatch):
    """The production FP8 arms with the output projection's dgrad fused into
    the LN * U * dropout backward (``outproj_lnmd_fused``) against the same
    layer unfused, with dropout: every gradient bit-equal except the output
    LayerNorm's weight and bias (fp32 sums in another fixed order: rtol 1e-5),
    which feed nothing upstream."""
    import hstu_amd
    import hstu_amd.bwd_fp8 as B

    monkeypatch.setattr(L_mod, "_mask16", True)
    lengths = np.array([300, 77, 512, 129])
    T, N, E = int(lengths.sum()), 512, 512
    g = torch.Generator().manual_seed(21)
    x = torch.randn(T, E, generator=g).to(torch.bfloat16)
    params = LO.make_layer_params(E, seed=6)
    s_x, s_qkv = _calibrate(x, params)
    dy = torch.randn(T, E, generator=g).to(torch.bfloat16)
    offs = orc.offsets_from_lengths(lengths).to(DEV)
    sc = (lambda s: torch.full((1, 1), s, device=DEV))
    grads = {}
    for fused in (False, True):
        cfg = B.Fp8BackwardConfig(enabled=True, uvqk=True, warmup_calls=1, uvqk_wgrad_fp8t=True,
                                  out_wgrad_fp8=True, outproj_lnmd_fused=fused)
        B.reset_sites()
        pd = {k: v.to(DEV).requires_grad_(True) for k, v in params.items()}
        for _ in range(2):                  # step 1 publishes the scales (bf16), step 2 runs FP8
            for t in pd.values():
                t.grad = None
            xd = x.to(DEV).requires_grad_(True)
            out = hstu_amd.hstu_layer(xd, offs, N, pd, dropout_ratio=0.3, training=True, fp8_input_scale=sc(s_x),
                                      fp8_qkv_scale=sc(s_qkv), fp8_output_scale=sc(0.05), fp8_backward=cfg, seed=5)
            out.backward(dy.to(DEV))
        grads[fused] = {"out": out.detach(), "dx": xd.grad, **{k: t.grad for k, t in pd.items()}}
    for name, ref in grads[False].items():
        got = grads[True][name]
        if name.startswith("output_norm"):
            torch.testing.assert_close(got.float(), ref.float(), rtol=1e-5, atol=1e-6 * float(ref.abs().max()),
                                       msg=name)
        else:
            assert torch.equal(got, ref), name
