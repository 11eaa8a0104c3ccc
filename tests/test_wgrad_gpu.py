"""The split-K token-axis wgrad kernel (hstu_wgrad) against the float64
oracle: a^T b of the same bf16 operands, and (sa a8)^T (sb b8) of the same
fp8 operands (e4m3 x e5m2 / e4m3).

Tolerances: fp32 output relative L2 <= 1e-5 for bf16 operands (bf16 products
are exact in fp32; only the fp32 summation order differs) and <= 1e-4 for fp8
operands (the f8f6f4 MFMA's internal summation); bf16 output relative L2 <= 4e-3 and
max |err| <= 2^-7 max |ref| (one bf16 rounding).  The fixed-order split
reduction is checked bitwise: two calls give the same bytes."""

import pytest
import torch

from oracle import hstu_bwd_fp8_oracle as O

pytestmark = pytest.mark.gpu


def _rel(ref, got):
    ref, got = ref.double(), got.double().cpu()
    return float((got - ref).norm() / ref.norm().clamp_min(1e-30))


@pytest.mark.parametrize("T,N1,N2,split", [(1000, 512, 2048, None), (5000, 1536, 512, None), (777, 256, 256, 1),
                                           (4099, 512, 512, 3), (1, 256, 512, None), (33, 768, 256, 7)])
def test_wgrad_against_fp64(hip_lib, T, N1, N2, split):
    from hstu_amd.wgrad import wgrad

    g = torch.Generator(device="cuda").manual_seed(T + N1)
    a = torch.randn(T, N1, device="cuda", generator=g).to(torch.bfloat16)
    b = torch.randn(T, N2, device="cuda", generator=g).to(torch.bfloat16)
    ref = O.wgrad(a, b)
    out32 = wgrad(a, b, out_dtype=torch.float32, split=split)
    assert out32.shape == (N1, N2) and out32.dtype == torch.float32
    assert _rel(ref, out32) <= 1e-5
    out16 = wgrad(a, b, split=split)
    assert _rel(ref, out16) <= 4e-3
    assert float((out16.double().cpu() - ref).abs().max()) <= 2.0 ** -7 * float(ref.abs().max())
    again = wgrad(a, b, split=split)
    assert torch.equal(out16, again)
    # the fused column sums of b: within the fp32 summation bound of the float64 sum
    out_c, cs = wgrad(a, b, split=split, with_colsum=True)
    assert torch.equal(out_c, out16)
    ref_cs = b.double().cpu().sum(0)
    bound = (T + 64) * 2.0 ** -24 * b.double().abs().cpu().sum(0) + 1e-30
    assert bool(((cs.double().cpu() - ref_cs).abs() <= bound).all())


def test_wgrad_strided_operands_scales_and_empty(hip_lib):
    """Column slices of wider buffers (the layer's d(uvqk) blocks), device
    scales, and T = 0 (zeros)."""
    from hstu_amd.wgrad import token_wgrad, wgrad

    g = torch.Generator(device="cuda").manual_seed(5)
    big_a = torch.randn(3001, 1024, device="cuda", generator=g).to(torch.bfloat16)
    big_b = torch.randn(3001, 2048, device="cuda", generator=g).to(torch.bfloat16)
    a, b = big_a[:, 256:768], big_b[:, 512:1536]
    sa = torch.tensor([0.5], device="cuda")
    sb = torch.tensor([3.0], device="cuda")
    out = wgrad(a, b, out_dtype=torch.float32, scale_a=sa, scale_b=sb)
    assert _rel(O.wgrad(a, b, 0.5, 3.0), out) <= 1e-5
    z = wgrad(a[:0], b[:0])
    assert z.shape == (512, 1024) and not bool(z.any())
    z, zc = wgrad(a[:0], b[:0], with_colsum=True)
    assert not bool(z.any()) and zc.shape == (1024,) and not bool(zc.any())
    _, cs = wgrad(a, b, with_colsum=True)                                    # strided b
    assert float((cs.double().cpu() - b.double().cpu().sum(0)).abs().max()) <= 1e-3
    # token_wgrad: the kernel for served shapes, torch.mm otherwise
    assert _rel(O.wgrad(a, b), token_wgrad(a, b)) <= 4e-3
    c = big_a[:, :300]
    assert _rel(O.wgrad(c, b), token_wgrad(c, b)) <= 4e-3


@pytest.mark.parametrize("bdt", [torch.float8_e5m2, torch.float8_e4m3fn])
@pytest.mark.parametrize("T,N1,N2,split", [(1000, 512, 2048, None), (3001, 1536, 512, None), (129, 256, 256, 1),
                                           (5000, 512, 768, 5)])
def test_fp8_wgrad_against_fp64(hip_lib, bdt, T, N1, N2, split):
    """The fp32 output is within 1e-4 relative L2 of the float64 product of
    the same fp8 values and scales: the f8f6f4 MFMA's own summation of its
    128 products rounds more than a plain fp32 chain (1.2e-5 measured at
    T = 1000, against 2e-6 for the bf16 MFMA)."""
    from hstu_amd.wgrad import fp8_wgrad

    g = torch.Generator(device="cuda").manual_seed(T + N2)
    a8 = (torch.randn(T, N1, device="cuda", generator=g) * 40).to(torch.float8_e4m3fn)
    # within each format's range (torch's e4m3 cast of |x| > 448 is NaN)
    b8 = (torch.randn(T, N2, device="cuda", generator=g) * (300 if bdt == torch.float8_e5m2 else 40)).to(bdt)
    sa = torch.tensor([0.01], device="cuda")
    sb = torch.tensor([0.002], device="cuda")
    ref = O.wgrad(a8, b8, 0.01, 0.002)
    out32 = fp8_wgrad(a8, b8, sa, sb, out_dtype=torch.float32, split=split)
    assert _rel(ref, out32) <= 1e-4
    out16 = fp8_wgrad(a8, b8, sa, sb, split=split)
    assert _rel(ref, out16) <= 4e-3
    assert torch.equal(out16, fp8_wgrad(a8, b8, sa, sb, split=split))
    # strided rows: column slices of wider fp8 buffers
    big = (torch.randn(T, N1 + 256, device="cuda", generator=g) * 40).to(torch.float8_e4m3fn)
    a_s = big[:, 256:]
    assert _rel(O.wgrad(a_s, b8, 0.01, 0.002), fp8_wgrad(a_s, b8, sa, sb, out_dtype=torch.float32)) <= 1e-4


@pytest.mark.parametrize("n1,n2", [(512, 2048), (1536, 512)])
def test_wgrad_full_size_against_fp32_library_product(hip_lib, n1, n2):
    """At the layer's full token count (config 3, T = 162 251, 16 or 21
    splits): the bf16 and e4m3 x e5m2 products against torch's fp32 matmul of
    the same values on the device (relative L2 1e-5 / 1e-4), and the fused
    column sums against torch's fp32 sum."""
    from hstu_amd.wgrad import fp8_wgrad, wgrad

    T = 162251
    g = torch.Generator(device="cuda").manual_seed(n1)
    a = torch.randn(T, n1, device="cuda", generator=g).to(torch.bfloat16)
    b = torch.randn(T, n2, device="cuda", generator=g).to(torch.bfloat16)
    ref = torch.mm(a.float().t(), b.float())
    out, cs = wgrad(a, b, out_dtype=torch.float32, with_colsum=True)
    assert float((out - ref).norm() / ref.norm()) <= 1e-5
    rcs = b.float().sum(0)
    # two fp32 summations of the same values: within (T + 64) 2^-24 sum|b| of each other, per column
    assert bool(((cs - rcs).abs() <= (T + 64) * 2.0 ** -24 * b.float().abs().sum(0)).all())
    a8, b8 = a.to(torch.float8_e4m3fn), b.to(torch.float8_e5m2)
    one = torch.ones(1, device="cuda")
    ref8 = torch.mm(a8.float().t(), b8.float())
    out8 = fp8_wgrad(a8, b8, one, one, out_dtype=torch.float32)
    assert float((out8 - ref8).norm() / ref8.norm()) <= 1e-4
