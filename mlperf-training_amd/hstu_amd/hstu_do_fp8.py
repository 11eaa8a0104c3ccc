"""dO -> e4m3 with power-of-two block scales, the input of the full-FP8
attention backward, on this build's kernel (``hstu_quantize_do_e4m3_blk``).

Drop-in for ``quantize_do_e4m3_blk`` (``ops/flydsl/hstu_do_fp8.py:95-121``,
reference paths relative to ``recommendation_v4/hstu/generative_recommenders/``):
one pow2 scale per (sequence, head, 32-token group), the groups being tokens
p % 16 < 8 and p % 16 >= 8 of each 64-token tile of a sequence; no host sync.
"""

from __future__ import annotations

from typing import Tuple

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
