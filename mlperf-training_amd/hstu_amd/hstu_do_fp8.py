"""dO -> e4m3 with power-of-two block scales, the input of the full-FP8
attention backward, on this build's kernel (``hstu_quantize_do_e4m3_blk``).

Drop-in for ``quantize_do_e4m3_blk`` (``ops/flydsl/hstu_do_fp8.py:95-121``,
reference paths relative to ``recommendation_v4/hstu/generative_recommenders/``):
one pow2 scale per (sequence, head, 32-token group), the groups being tokens
p % 16 < 8 and p % 16 >= 8 of each 64-token tile of a sequence; no host sync.

``bwd_full_fp8_enabled`` reads the reference's switch ``DLRM_HSTU_FP8_BWD_FULL``
(``hstu_flydsl_mha.py:458-464``).  Under it the FP8 attention backward runs on
the block-quantized dO: ``quantize_do_e4m3_blk`` then the exact
``dequantize_do_e4m3_blk``, so its gradients are those of the reference's
contract for the dO operand (the reference undoes the scales inside its
MFMAs, :1330-1394).  The e4m3 P / dS operands of that backward are not built.
"""

from __future__ import annotations

import os
from typing import Optional, Tuple

import torch

from . import _lib


def quantize_do_e4m3_blk(dout: torch.Tensor, seq_offsets: torch.Tensor, N: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """dout [T, H, D] bf16/fp32, seq_offsets [B+1], N >= every sequence length.
    Returns (dO8 [T, H, D] float8_e4m3fn, E8 [T, H] uint8 = 127 - e)."""
    if dout.dim() != 3:
        raise ValueError("dout must be [T, H, D]")
    T, H, D = dout.shape
    if dout.dtype == torch.bfloat16:
        dt = _lib.HSTU_DTYPE_BF16
    elif dout.dtype == torch.float32:
        dt = _lib.HSTU_DTYPE_FP32
    else:
        raise NotImplementedError(f"dO block quantizer serves bf16 / fp32, not {dout.dtype}")
    x = dout
    if x.stride(2) != 1 or x.stride(1) != D or x.data_ptr() % 16 or (x.stride(0) * x.element_size()) % 16:
        x = x.contiguous()
    y = torch.empty((T, H, D), dtype=torch.float8_e4m3fn, device=dout.device)
    e8 = torch.empty((T, H), dtype=torch.uint8, device=dout.device)
    B = seq_offsets.numel() - 1
    if B <= 0 or T == 0:
        return y, e8
    offs = seq_offsets.to(device=dout.device, dtype=torch.int64).contiguous()
    st = _lib.fn("hstu_quantize_do_e4m3_blk")(
        dt, x.data_ptr(), x.stride(0), offs.data_ptr(), B, H, D, int(N), y.data_ptr(), e8.data_ptr(),
        torch.cuda.current_stream(dout.device).cuda_stream)
    _lib.check(st, "hstu_quantize_do_e4m3_blk")
    return y, e8


_full: Optional[bool] = None


def bwd_full_fp8_enabled() -> bool:
    """The process default for the full-FP8 backward: ``DLRM_HSTU_FP8_BWD_FULL``
    in (1, true, on, yes), read once."""
    global _full
    if _full is None:
        _full = os.environ.get("DLRM_HSTU_FP8_BWD_FULL", "0").strip().lower() in ("1", "true", "on", "yes")
    return _full


def set_bwd_full_fp8(flag: Optional[bool]) -> None:
    """Set the full-FP8 backward default (None: read the environment again on next use)."""
    global _full
    _full = flag


def dequantize_do_e4m3_blk(dout8: torch.Tensor, e8: torch.Tensor) -> torch.Tensor:
    """bf16 [T, H, D] = dout8 * 2^(E8 - 127), exact."""
    if dout8.dim() != 3 or dout8.dtype != torch.float8_e4m3fn or e8.dtype != torch.uint8:
        raise ValueError("expected dO8 e4m3 [T, H, D] and E8 uint8 [T, H]")
    T, H, D = dout8.shape
    y = dout8.contiguous()
    e = e8.contiguous()
    out = torch.empty((T, H, D), dtype=torch.bfloat16, device=dout8.device)
    if T == 0:
        return out
    st = _lib.fn("hstu_dequantize_do_e4m3_blk")(y.data_ptr(), e.data_ptr(), T, H, D, out.data_ptr(), H * D,
                                                torch.cuda.current_stream(dout8.device).cuda_stream)
    _lib.check(st, "hstu_dequantize_do_e4m3_blk")
    return out


def block_quantized_do(dout: torch.Tensor, seq_offsets: torch.Tensor, N: int) -> torch.Tensor:
    """dO as the full-FP8 backward sees it: dequantize(quantize(dO)), bf16."""
    y, e8 = quantize_do_e4m3_blk(dout, seq_offsets, N)
    return dequantize_do_e4m3_blk(y, e8)
