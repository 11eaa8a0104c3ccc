"""dO -> e4m3 with power-of-two block scales, the input of the full-FP8
attention backward, on this build's kernel (``hstu_quantize_do_e4m3_blk``).

Drop-in for ``quantize_do_e4m3_blk`` (``ops/flydsl/hstu_do_fp8.py:95-121``,
reference paths relative to ``recommendation_v4/hstu/generative_recommenders/``):
one pow2 scale per (sequence, head, 32-token group), the groups being tokens
p % 16 < 8 and p % 16 >= 8 of each 64-token tile of a sequence; no host sync.

``bwd_full_fp8_enabled`` reads the reference's switch ``DLRM_HSTU_FP8_BWD_FULL``
(``hstu_flydsl_mha.py:458-464``).  Under it the FP8 attention backward runs
the full-FP8 kernels on ``quantize_do_e4m3_blk``'s output, with the e4m3 P
and dS pre-scales of ``full_fp8_prescale_log2``; for the masks those kernels
do not serve it runs the e4m3-input backward on the exact
``dequantize_do_e4m3_blk`` of the quantized dO.
"""

from __future__ import annotations

import math
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


SSC_K_DEFAULT = 3
DSC_K_DEFAULT = -3


def full_fp8_prescale_log2(N: int, *, ssc_k: Optional[int] = None, dsc_k: Optional[int] = None) -> Tuple[int, int]:
    """(P, dS) e4m3 pre-scale exponents of the full-FP8 backward, as the
    reference resolves them per call (``hstu_flydsl_mha.py:1351-1374``): with
    c = ceil(log2 max(N, 2)), ``DLRM_HSTU_FP8_BWD_FULL_{SSC,DSC}_LOG2`` (an
    absolute exponent) if set, else c + ``DLRM_HSTU_FP8_BWD_FULL_{SSC,DSC}_K``
    (defaults 3 and -3; the production gin sets DSC_K = -5,
    ``yambda_5b.gin:3799``).  ``ssc_k`` / ``dsc_k`` given (the layer's
    ``Fp8BackwardConfig``) replace the environment.  The P exponent may not
    exceed c + 9 (the SiLU's upper-only clamp stays exact below it)."""
    c = int(math.ceil(math.log2(max(int(N), 2))))

    def one(name: str, k: Optional[int], k_default: int) -> int:
        if k is not None:
            return c + int(k)
        ab = os.environ.get(f"DLRM_HSTU_FP8_BWD_FULL_{name}_LOG2")
        if ab not in (None, ""):
            return int(ab)
        return c + int(os.environ.get(f"DLRM_HSTU_FP8_BWD_FULL_{name}_K", str(k_default)))

    e_p, e_ds = one("SSC", ssc_k, SSC_K_DEFAULT), one("DSC", dsc_k, DSC_K_DEFAULT)
    if e_p > c + 9:
        raise ValueError(f"full-FP8 backward: P pre-scale 2^{e_p} above 2^(ceil(log2 N) + 9) = 2^{c + 9}")
    if not (-64 <= e_p <= 64 and -64 <= e_ds <= 64):
        raise ValueError(f"full-FP8 backward: pre-scale exponents ({e_p}, {e_ds}) outside [-64, 64]")
    return e_p, e_ds


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
