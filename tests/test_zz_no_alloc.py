"""The allocation-free forward (hstu_attn_fwd_noalloc) through the C ABI:
its output equals hstu_attn_fwd's bitwise (the same kernels; only where the
block schedule lives differs), on two calls in a row with the second one
smaller, for bf16 inputs and for e4m3 inputs with per-(token, head) scales
and the relative bias."""

import ctypes

import numpy as np
import pytest
import torch

from oracle import hstu_oracle as orc

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _ptr(t):
    return None if t is None else t.data_ptr()


def _call(lib, name, dtype, q, k, v, scales, offs, N, alpha, bias, R, out):
    T, H, D = q.shape
    B = offs.numel() - 1
    stream = torch.cuda.current_stream().cuda_stream
    qs, ks, vs = scales if scales is not None else (None, None, None)
    srs, shs = (H, 1) if scales is not None else (0, 0)
    common = [dtype, q.data_ptr(), k.data_ptr(), v.data_ptr(), H * D, H * D, H * D, _ptr(qs), _ptr(ks), _ptr(vs),
              srs, shs, offs.data_ptr(), B, H, D, N, alpha, None, 0, 0, _ptr(bias), R, out.data_ptr(), H * D]
    if name == "hstu_attn_fwd":
        nbytes = lib.fn("hstu_attn_fwd_workspace_bytes")(dtype, T, B, H, D, N)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
        st = lib.fn(name)(*common, ws.data_ptr(), nbytes, T, stream)
    else:
        st = lib.fn(name)(*common, T, stream)
    torch.cuda.synchronize()
    assert st == 0, f"{name} returned {st}"
    return out


@pytest.mark.parametrize("fp8", [False, True])
def test_noalloc_forward_matches_workspace_forward(hip_lib, fp8):
    import hstu_amd._lib as lib

    H, D = 4, 128
    alpha = 1.0 / D ** 0.5
    for call, lengths in enumerate(([700, 33, 1024, 129, 1, 300, 64, 511], [97, 260, 5])):
        print(f"noalloc call {call}: fp8={fp8} lengths={lengths}", flush=True)
        N = max(lengths)
        q, k, v = orc.make_qkv(lengths, H, D, 1.0 if fp8 else 0.5, seed=call)
        offs = orc.offsets_from_lengths(lengths).to(DEV)
        if fp8:
            (q8, sq), (k8, sk), (v8, sv) = (orc.quantize_e4m3_rows(t, dim=-1) for t in (q, k, v))
            qd, kd, vd = (t.to(DEV) for t in (q8, k8, v8))
            scales = tuple(s.to(DEV).float().contiguous() for s in (sq, sk, sv))
            bias = orc.make_bias(H, 1024).to(DEV).float().contiguous()
            R, dtype = 1024, lib.HSTU_DTYPE_FP8_E4M3
        else:
            qd, kd, vd = (t.to(torch.bfloat16).to(DEV) for t in (q, k, v))
            scales, bias, R, dtype = None, None, 0, lib.HSTU_DTYPE_BF16
        want = torch.full((q.shape[0], H, D), float("nan"), dtype=torch.bfloat16, device=DEV)
        got = torch.full_like(want, float("nan"))
        _call(lib, "hstu_attn_fwd", dtype, qd, kd, vd, scales, offs, N, alpha, bias, R, want)
        _call(lib, "hstu_attn_fwd_noalloc", dtype, qd, kd, vd, scales, offs, N, alpha, bias, R, got)
        assert not torch.isnan(got.float()).any()
        assert torch.equal(got, want), f"call {call}: outputs differ"
