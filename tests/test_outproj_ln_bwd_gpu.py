"""GPU parity of the fused output-projection backward (``hstu_outproj_ln_bwd``:
the e5m2 x e4m3 dgrad dy = g8 . w8^T * s_g s_w fused with the LN * U *
dropout backward of the [u' | x | y] concat), through the HIP C ABI.

Bars:
* dx, du: bit-equal to the unfused pair on the same inputs -- ``hstu_fp8_gemm``
  (the e5m2 dgrad, bf16 dy in HBM) then ``hstu_ln_mul_bwd`` (same MFMAs,
  operand bytes, epilogue and row code, so any difference is a bug);
* dweight / dbias: fp32 sums in another fixed order than the unfused path's:
  rtol 1e-5, atol 1e-6 max |ref| against it; bit-equal run to run;
* against the float64 oracle (dy = the dequantized product rounded to bf16,
  then ``oracle/hstu_ln_oracle.ln_mul_dropout_bwd``): the bf16 bar of
  tests/test_ln_gpu.py (assert_close rtol = atol = 1e-2, relative L2 <= 4e-3).
"""

import pytest
import torch

import hstu_amd.hstu_linear as L_mod
from hstu_amd import bwd_fp8

from oracle import hstu_ln_oracle as L

pytestmark = pytest.mark.gpu

DEV = "cuda"
D = 512


def _ops():
    import hstu_amd

    return hstu_amd


def _case(N, seed=0, training=True, act="silu", p=0.3):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(N, D, generator=g) * 1.5 + 0.3).to(torch.bfloat16)
    u = torch.randn(N, D, generator=g).to(torch.bfloat16)
    w = (1.0 + 0.2 * torch.randn(D, generator=g)).to(torch.bfloat16)
    b = (0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    g8 = (torch.randn(N, D, generator=g) * 3.0).to(torch.float8_e5m2)
    w8 = (torch.randn(3 * D, D, generator=g) * 60.0).clamp(-448, 448).to(torch.float8_e4m3fn)
    gs = torch.tensor([0.0123], dtype=torch.float32)
    ws = torch.tensor([0.0071], dtype=torch.float32)
    xd, ud, wd, bd = (t.to(DEV) for t in (x, u, w, b))
    _, mean, rstd, _, _, _, mask = _ops().triton_layer_norm_mul_dropout_fwd(
        xd, ud, wd, bd, 1e-6, p, training, True, True, True, act, 17)
    return dict(x=xd, u=ud, w=wd, b=bd, g8=g8.to(DEV), w8=w8.to(DEV), gs=gs.to(DEV), ws=ws.to(DEV), mean=mean,
                rstd=rstd, mask=mask, p=p if training else 0.0, act=act, cpu=(x, u, w, b, g8, w8, gs, ws))


def _unfused(c, du_row_width=2048):
    dy = bwd_fp8.fp8_dgrad(c["g8"], c["gs"], c["w8"], c["ws"])
    dx, du, dw, db, _ = L_mod._ln_bwd(dy, c["x"], c["u"], c["w"], c["b"], c["mean"], c["rstd"], c["p"], c["mask"],
                                      True, True, True, c["act"], False, du_row_width)
    return dy, dx, du, dw, db


def _fused(c, du_row_width=2048):
    return L_mod._outproj_ln_bwd(c["g8"], c["gs"], c["w8"], c["ws"], c["x"], c["u"], c["w"], c["b"], c["mean"],
                                 c["rstd"], c["p"], c["mask"], True, c["act"], du_row_width)


def _check_equal(c, what):
    _, rdx, rdu, rdw, rdb = _unfused(c)
    dx, du, dw, db = _fused(c)
    torch.cuda.synchronize()
    assert torch.equal(dx, rdx), f"{what}: dx differs from the unfused path"
    assert torch.equal(du, rdu), f"{what}: du differs from the unfused path"
    for name, got, ref in (("dweight", dw, rdw), ("dbias", db, rdb)):
        torch.testing.assert_close(got, ref, rtol=1e-5, atol=1e-6 * float(ref.abs().max()), msg=f"{what}: {name}")
    return dx, du, dw, db


@pytest.mark.parametrize("N", [1, 63, 64, 65, 1000, 20000])
def test_fused_equals_unfused(hip_lib, N):
    """Ragged last blocks (63, 65), one block, and more blocks than
    workgroups (20000 rows = 313 blocks over 256 workgroups)."""
    print(f"fused out-proj backward: N={N}", flush=True)
    _check_equal(_case(N, seed=N), f"N={N}")


@pytest.mark.parametrize("act,training", [("silu", False), ("none", True), ("sigmoid", True)])
def test_fused_equals_unfused_variants(hip_lib, act, training):
    print(f"fused out-proj backward: act={act} training={training}", flush=True)
    _check_equal(_case(777, seed=3, training=training, act=act), f"act={act} training={training}")


def test_fused_deterministic_and_du_row(hip_lib):
    c = _case(3001, seed=9)
    a = _fused(c)
    b = _fused(c, du_row_width=0)
    torch.cuda.synchronize()
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    assert a[1].stride(0) == 2048 and b[1].stride(0) == D


def test_fused_against_oracle(hip_lib):
    N, p = 300, 0.3
    c = _case(N, seed=5)
    dx, du, dw, db = _fused(c)
    x, u, w, b, g8, w8, gs, ws = c["cpu"]
    dy = ((g8.double() * float(gs)) @ (w8.double() * float(ws)).t()).to(torch.bfloat16).double()
    rdx, rdu, rdw, rdb = L.ln_mul_dropout_bwd(dy, x.double(), u.double(), w.double(), b.double(), 1e-6,
                                              dropout_ratio=p, mask=c["mask"].cpu().numpy().astype("uint8"),
                                              silu_u=True, concat_u=True, concat_x=True,
                                              mul_u_activation_type="silu")
    for name, got, ref in (("dx", dx, rdx), ("du", du, rdu)):
        got = got.float().cpu()
        torch.testing.assert_close(got, ref.float(), rtol=1e-2, atol=1e-2, msg=name)
        rel = float((got.double() - ref).norm() / ref.norm())
        assert rel <= 4e-3, (name, rel)
    for name, got, ref in (("dweight", dw, rdw), ("dbias", db, rdb)):
        torch.testing.assert_close(got.double().cpu(), ref, rtol=5e-3, atol=1e-3 * float(ref.abs().max()), msg=name)


def test_fused_config3_rows(hip_lib):
    """Config 3's 162 251 tokens: bit-equal to the unfused pair."""
    print("fused out-proj backward: config 3 rows", flush=True)
    _check_equal(_case(162251, seed=1), "config 3 rows")


def test_fused_strided_operands(hip_lib):
    """Column slices of wider buffers (as the layer hands them over): x from
    [N, 1024], u from [N, 2048], the e5m2 gradient from [N, 1024] bytes; bit-equal
    to the unfused pair on the same views."""
    N = 1500
    c = _case(N, seed=12)
    xs = torch.zeros(N, 1024, dtype=torch.bfloat16, device=DEV)
    us = torch.zeros(N, 2048, dtype=torch.bfloat16, device=DEV)
    gs8 = torch.zeros(N, 1024, dtype=torch.float8_e5m2, device=DEV)
    xs[:, 256:768] = c["x"]
    us[:, 1024:1536] = c["u"]
    gs8[:, 512:] = c["g8"]
    c.update(x=xs[:, 256:768], u=us[:, 1024:1536], g8=gs8[:, 512:])
    assert c["x"].stride(0) == 1024 and c["u"].stride(0) == 2048 and c["g8"].stride(0) == 1024
    ref = _unfused(c)
    got = _fused(c)
    torch.cuda.synchronize()
    assert torch.equal(got[0], ref[1]) and torch.equal(got[1], ref[2])
