"""The FP8 e4m3-output projection GEMM against the reference's own K=512
kernel, built from its source into ``oracle/_ref`` by ``oracle/build_ref.py``
(``ops/hip/k512_fp8_gemm.cu``, entry ``k512_fp8_gemm_e4m3_bias_N1536``,
:555-558): C = e4m3_rne(sat448(acc * (sa * sb) + bias[n])) with fp32
accumulation over four in-order K = 128 steps and one rounding after the
multiply and one after the add (its header, :13-17).

This build's ``hstu_fp8_gemm_rowcol`` with per-tensor scales, an output
scale of 1 and the same bf16 bias must give the same bytes: bitwise equality
on ragged M (1, 129, 1000), config 3's token count and config 4's M = 262 144,
with values that saturate at +-448 included.  Skipped where the reference
tree was absent when the library was built (nothing in ``oracle/_ref``).
"""

import ctypes
from pathlib import Path

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"
REF_SO = Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "libk512_fp8_gemm_n1536.so"
N, K = 1536, 512


@pytest.fixture(scope="module")
def ref_lib():
    if not REF_SO.exists():
        pytest.skip("oracle/_ref/libk512_fp8_gemm_n1536.so not built (no reference tree at build time)")
    lib = ctypes.CDLL(str(REF_SO))
    f = lib.k512_fp8_gemm_e4m3_bias_N1536
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_void_p] * 6 + [ctypes.c_int, ctypes.c_void_p]
    return f


@pytest.mark.parametrize("M", [1, 129, 1000, 162251, 262144])
def test_e4m3_out_gemm_bitwise_vs_reference_kernel(hip_lib, ref_lib, M):
    import hstu_amd._lib as L

    g = torch.Generator(device=DEV).manual_seed(M)
    a8 = (torch.randn(M, K, device=DEV, generator=g) * 40).clamp(-448, 448).to(torch.float8_e4m3fn)
    w8 = (torch.randn(N, K, device=DEV, generator=g) * 40).clamp(-448, 448).to(torch.float8_e4m3fn)
    bias = (torch.randn(N, device=DEV, generator=g) * 8).to(torch.bfloat16)
    # |acc| ~ 40 * 40 * sqrt(512) ~ 3.6e4: sa * sb = 6e-3 puts outputs around 200, a few % past 448
    sa = torch.tensor([0.075], device=DEV)
    sb = torch.tensor([0.08], device=DEV)
    one = torch.ones(1, device=DEV)
    c_ref = torch.full((M, N), 0x55, dtype=torch.uint8, device=DEV)
    c_our = torch.full((M, N), 0xAA, dtype=torch.uint8, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    print(f"k512 reference vs hstu_fp8_gemm_rowcol: M={M}", flush=True)
    assert ref_lib(a8.data_ptr(), w8.data_ptr(), c_ref.data_ptr(), bias.data_ptr(), sa.data_ptr(), sb.data_ptr(),
                   M, stream) == 0
    st = L.fn("hstu_fp8_gemm_rowcol")(a8.data_ptr(), K, w8.data_ptr(), K, sa.data_ptr(), 0, sb.data_ptr(), 0,
                                     bias.data_ptr(), None, 0, c_our.data_ptr(), N, L.HSTU_DTYPE_FP8_E4M3,
                                     one.data_ptr(), M, N, K, 0, 0, stream)
    L.check(st, "hstu_fp8_gemm_rowcol")
    torch.cuda.synchronize()
    sat = (c_ref.view(torch.float8_e4m3fn).float().abs() == 448).float().mean().item()
    mism = (c_ref != c_our).sum().item()
    print(f"  saturated fraction {sat:.2e}, mismatching bytes {mism}", flush=True)
    assert mism == 0, f"{mism} of {M * N} bytes differ from the reference kernel"
    if M >= 1000:
        assert sat > 1e-3, "the inputs should reach the saturation at 448"
