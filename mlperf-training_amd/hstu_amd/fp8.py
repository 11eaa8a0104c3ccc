"""FP8 (OCP e4m3) quantization and projection GEMMs of the HSTU layer on the
gfx950 kernels of ``libhstu_mi355x.so``.

Mirrors the reference's FP8 boundary (``ops/triton/triton_fp8.py``, paths
relative to ``recommendation_v4/hstu/generative_recommenders/``):

* ``quantize_with_scale`` (:760-781) / ``calibrated_scale`` (:396-413)
  -> ``quantize_with_scale`` / ``quantize_e4m3_rows`` (also per row and per
  (token, head) groups, which the reference does not have);
* the per-layer FP8 scale state ``[scale, completed, amax history]``
  (``fp8_scale_state_size`` :346-349, ``fp8_scale_tensor`` :352-355,
  ``calibrate_scale_buffer`` :694-749, ``modules/stu.py:317-328``) ->
  the same functions, plus ``scale_ready`` (is a scale usable now, known on the
  host without a device read once the state is frozen);
* ``scaled_addmm_fp8_preq`` (:1756) -> ``scaled_addmm_fp8_preq`` (bf16 out,
  bias or residual);
* ``scaled_mm_fp8_out_preq`` (:2409) -> ``scaled_mm_fp8_out_preq`` (e4m3 out
  at an output scale, the VQK projection feeding the FP8 attention).

Weights are passed as bf16 ``[K, N]`` (the layer's parameter layout) or as a
pre-quantized ``(w8_nk, w_scale)`` pair from ``quantize_weight_e4m3``.
"""

from __future__ import annotations

import math
import os
import weakref
from typing import Dict, Optional, Tuple, Union

import torch

from . import _lib

E4M3 = torch.float8_e4m3fn
E4M3_MAX = 448.0
# The reference's defaults (``triton_fp8.py:96-101``), read once at import as it does.
ASCALE_MARGIN = float(os.environ.get("DLRM_HSTU_FP8_GEMM_ASCALE_MARGIN", "1.5"))
CALIBRATION_STEPS = max(1, int(os.environ.get("DLRM_HSTU_FP8_CALIBRATION_STEPS", "4")))
Weight = Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]]


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def quantize_e4m3_rows(x: torch.Tensor, group: Optional[int] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """bf16 [R, C] (or [T, H, D] with group=D) -> (e4m3 same shape, fp32 scales
    [R, C/group]); scale = amax/448 per group of ``group`` consecutive
    elements of a row (default: the whole row)."""
    shape = x.shape
    x2 = x.reshape(shape[0], -1)
    if x2.dtype != torch.bfloat16:
        x2 = x2.to(torch.bfloat16)
    x2 = x2.contiguous()
    R, C = x2.shape
    group = C if group is None else int(group)
    out = torch.empty((R, C), dtype=E4M3, device=x.device)
    scales = torch.empty((R, C // group), dtype=torch.float32, device=x.device)
    st = _lib.fn("hstu_quantize_e4m3_rows")(x2.data_ptr(), C, R, C, group, None, out.data_ptr(), C,
                                            scales.data_ptr(), _stream(x))
    _lib.check(st, "hstu_quantize_e4m3_rows")
    return out.view(shape), scales


def quantize_with_scale(value: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """e4m3(clamp(value / scale, +-448)) with one per-tensor fp32 scale
    (``quantize_with_scale``, ``triton_fp8.py:760-781``)."""
    x2 = value.reshape(value.shape[0], -1).to(torch.bfloat16).contiguous()
    R, C = x2.shape
    group = C if C <= 4096 else next(g for g in (4096, 2048, 1024, 512, 256, 128, 64, 32, 16, 8) if C % g == 0)
    out = torch.empty((R, C), dtype=E4M3, device=value.device)
    s = scale.reshape(1).to(torch.float32).contiguous()
    st = _lib.fn("hstu_quantize_e4m3_rows")(x2.data_ptr(), C, R, C, group, s.data_ptr(), out.data_ptr(), C,
                                            None, _stream(value))
    _lib.check(st, "hstu_quantize_with_scale")
    return out.view(value.shape)


def calibrated_scale(value: torch.Tensor, *, margin: Optional[float] = None,
                     fp8_max: float = E4M3_MAX) -> torch.Tensor:
    """Per-tensor scale amax*margin/fp8_max as a (1, 1) fp32 tensor, margin
    1.5 by default (``calibrated_scale``, ``triton_fp8.py:396-413``)."""
    m = ASCALE_MARGIN if margin is None else margin
    amax = value.detach().abs().amax().float().clamp_min(1.0e-12)
    return (amax * m / fp8_max).reshape(1, 1)


# ---------------------------------------------------------------------------
# per-layer scale state: [scale, completed calibration steps, amax history]
# ---------------------------------------------------------------------------
def fp8_scale_state_size() -> int:
    """Length of one scale state buffer: scale, completed count, history."""
    return 2 + CALIBRATION_STEPS


def fp8_scale_tensor(scale_state: torch.Tensor) -> torch.Tensor:
    """The (1, 1) scale view of a state buffer (or of a plain scale)."""
    if scale_state.numel() < 1:
        raise ValueError("FP8 scale state cannot be empty")
    return scale_state.reshape(-1)[:1].reshape(1, 1)


# Host knowledge of each scale tensor: storage address -> (version counter
# when last seen, completed steps, the tensor itself as a weak reference).
# Tensors this module updates stay known without reading the device; a
# tensor changed elsewhere (loaded from a checkpoint, reset), or a new tensor
# on a recycled address, is read once.
_known: Dict[Tuple[int, int], Tuple[int, int, "weakref.ref"]] = {}


def _key(buf: torch.Tensor) -> Tuple[int, int]:
    return buf.untyped_storage().data_ptr(), buf.storage_offset()


def _completed(buf: torch.Tensor) -> int:
    """Completed calibration steps of a state buffer; for a one-element scale
    1 once its value is finite and positive (the reference's
    ``activation_scale_value``, ``triton_fp8.py:429-442``), else 0."""
    key = _key(buf)
    seen = _known.get(key)
    if seen is not None and seen[0] == buf._version and seen[2]() is buf:
        return seen[1]
    flat = buf.reshape(-1)
    if flat.numel() >= 3:
        done = int(flat[1].item())
    else:
        v = float(flat[0].item())
        done = 1 if math.isfinite(v) and v > 0.0 else 0
    _remember(buf, done)
    return done


def _remember(buf: torch.Tensor, done: int) -> None:
    _known[_key(buf)] = (buf._version, done, weakref.ref(buf))


def scale_ready(scale: Optional[torch.Tensor]) -> bool:
    """Can the FP8 path use this scale now?  A one-element tensor is a plain
    scale, usable once its value is finite and positive (read once per
    tensor and version: a zero or non-finite scale runs bf16 and is
    calibrated, as the reference's ``activation_scale_value`` returns None
    for it); a state buffer is usable once its calibration window is
    complete.  No device read for a tensor this module calibrated."""
    if scale is None:
        return False
    if scale.numel() == 1:
        return _completed(scale) >= 1
    if scale.numel() < 3:
        raise ValueError("FP8 scale state must contain scale, count, and amax history")
    return _completed(scale) >= scale.numel() - 2


def calibrate_scale_buffer(scale_buffer: torch.Tensor, value: torch.Tensor, *, margin: Optional[float] = None,
                           synchronize: bool = True) -> float:
    """One calibration step of a scale state (``calibrate_scale_buffer``,
    ``triton_fp8.py:694-749``): this call's amax joins the history; once the
    history is full the scale is max(history) * margin / 448 and stays there
    (the state is frozen).  A one-element buffer is simply set from this
    call.  Both scales are the reference's device expression
    ``amax * margin / 448`` in its operation order, so they match its bits.
    Returns the scale (0.0 while calibrating).  An all-zero value is not a
    step.  With torch.distributed initialised (world > 1) the amax is
    MAX-reduced across ranks first.  Bounded warm-up work: it reads the amax
    on the host, as the reference does; a frozen state returns at once."""
    m = ASCALE_MARGIN if margin is None else margin
    flat = scale_buffer.reshape(-1)
    if flat.numel() >= 3 and _completed(scale_buffer) >= flat.numel() - 2:
        return float(flat[0].item())
    amax = (value.detach().abs().amax().float() if value.numel()
            else torch.zeros((), dtype=torch.float32, device=scale_buffer.device))
    if (synchronize and torch.distributed.is_available() and torch.distributed.is_initialized()
            and torch.distributed.get_world_size() > 1):
        torch.distributed.all_reduce(amax, op=torch.distributed.ReduceOp.MAX)
    if not float(amax.item()) > 0.0:
        return float(flat[0].item()) if flat.numel() else 0.0
    amax = amax.to(scale_buffer.device).clamp_min(1.0e-12)
    if flat.numel() == 1:
        flat[:1].copy_((amax * m / E4M3_MAX).reshape(1))
        _remember(scale_buffer, 1)
        return float(flat[0].item())
    if flat.numel() < 3:
        raise ValueError("FP8 scale state must contain scale, count, and amax history")
    steps = flat.numel() - 2
    done = min(_completed(scale_buffer), steps)
    flat[2 + done].copy_(amax)
    done += 1
    flat[1].fill_(float(done))
    if done < steps:
        flat[0].zero_()
        _remember(scale_buffer, done)
        return 0.0
    flat[0].copy_(flat[2:2 + done].amax() * m / E4M3_MAX)
    _remember(scale_buffer, done)
    return float(flat[0].item())


def quantize_weight_e4m3(w_kn: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """bf16 weight [K, N] -> (e4m3 [N, K] row-major, per-column scales [N])."""
    w8, s = quantize_e4m3_rows(w_kn.t().contiguous())
    return w8, s.reshape(-1)


def _weight(weight: Weight) -> Tuple[torch.Tensor, torch.Tensor, int]:
    if isinstance(weight, tuple):
        w8, ws = weight
    else:
        w8, ws = quantize_weight_e4m3(weight)
    ws = ws.to(torch.float32).contiguous()
    return w8, ws, 1 if ws.numel() > 1 else 0


def fp8_gemm(a8: torch.Tensor, a_scale: torch.Tensor, weight: Weight, *, bias: Optional[torch.Tensor] = None,
             residual: Optional[torch.Tensor] = None, out_dtype: torch.dtype = torch.bfloat16,
             out_scale: Optional[torch.Tensor] = None,
             silu_cols: Optional[Tuple[int, int]] = None) -> torch.Tensor:
    """C = epilogue(a8 @ W^T) on the HIP kernel; see ``hstu_fp8_gemm_rowcol``."""
    if a8.dtype != E4M3:
        raise TypeError(f"expected e4m3 activation, got {a8.dtype}")
    w8, ws, w_mode = _weight(weight)
    M, K = a8.shape
    N = w8.shape[0]
    if w8.shape[1] != K:
        raise ValueError(f"K mismatch: a {tuple(a8.shape)} w8 {tuple(w8.shape)}")
    a8 = a8.contiguous()
    a_scale = a_scale.to(torch.float32).contiguous().reshape(-1)
    a_mode = 1 if a_scale.numel() > 1 else 0
    if a_mode and a_scale.numel() != M:
        raise ValueError("per-row activation scale must have M entries")
    fp8_out = out_dtype == E4M3
    out = torch.empty((M, N), dtype=out_dtype, device=a8.device)
    if M == 0:
        return out
    b = None if bias is None else bias.to(torch.bfloat16).contiguous()
    r = None if residual is None else residual.to(torch.bfloat16).contiguous()
    os_ = None
    if fp8_out:
        if out_scale is None:
            raise ValueError("e4m3 output needs out_scale")
        os_ = out_scale.to(torch.float32).reshape(1).contiguous()
    c0, c1 = silu_cols if silu_cols is not None else (0, 0)
    st = _lib.fn("hstu_fp8_gemm_rowcol")(
        a8.data_ptr(), K, w8.data_ptr(), w8.stride(0), a_scale.data_ptr(), a_mode, ws.data_ptr(), w_mode,
        _lib.ptr(b), _lib.ptr(r), N if r is not None else 0, out.data_ptr(), N,
        _lib.HSTU_DTYPE_FP8_E4M3 if fp8_out else _lib.HSTU_DTYPE_BF16, _lib.ptr(os_),
        M, N, K, int(c0), int(c1), _stream(a8))
    _lib.check(st, "hstu_fp8_gemm_rowcol")
    return out


def bf16_gemm(a: torch.Tensor, w_nk: torch.Tensor, *, bias: Optional[torch.Tensor] = None,
              residual: Optional[torch.Tensor] = None, silu_cols: Optional[Tuple[int, int]] = None,
              out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """bf16 C = epilogue(a @ w_nk^T) on the HIP tile kernel (``hstu_bf16_gemm``):
    a [M, K], w_nk [N, K] (the weight with the contraction index contiguous),
    optional bf16 bias [N], residual [M, N], SiLU on a column range.  ``out``:
    an [M, N] bf16 destination with unit column stride (e.g. columns of a
    wider buffer)."""
    if a.dtype != torch.bfloat16 or w_nk.dtype != torch.bfloat16:
        raise TypeError(f"expected bf16 operands, got {a.dtype} and {w_nk.dtype}")
    if a.stride(-1) != 1 or a.stride(0) % 8 != 0 or a.data_ptr() % 16 != 0:
        a = a.contiguous()
    if w_nk.stride(-1) != 1 or w_nk.stride(0) % 8 != 0 or w_nk.data_ptr() % 16 != 0:
        w_nk = w_nk.contiguous()
    M, K = a.shape
    N = w_nk.shape[0]
    if w_nk.shape[1] != K:
        raise ValueError(f"K mismatch: a {tuple(a.shape)} w {tuple(w_nk.shape)}")
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=a.device)
    elif out.shape != (M, N) or out.dtype != torch.bfloat16 or out.stride(1) != 1:
        raise ValueError("out must be a bf16 [M, N] view with unit column stride")
    if M == 0:
        return out
    b = None if bias is None else bias.to(torch.bfloat16).contiguous()
    r = None if residual is None else residual.to(torch.bfloat16).contiguous()
    c0, c1 = silu_cols if silu_cols is not None else (0, 0)
    st = _lib.fn("hstu_bf16_gemm")(a.data_ptr(), a.stride(0), w_nk.data_ptr(), w_nk.stride(0), _lib.ptr(b),
                                   _lib.ptr(r), N if r is not None else 0, out.data_ptr(), out.stride(0), M, N, K,
                                   int(c0), int(c1), _stream(a))
    _lib.check(st, "hstu_bf16_gemm")
    return out


def proj_mm(a: torch.Tensor, w_nk: torch.Tensor, *, bias: Optional[torch.Tensor] = None,
            residual: Optional[torch.Tensor] = None) -> torch.Tensor:
    """a @ w_nk^T (+ bias) (+ residual) for the layer's projections: the HIP
    bf16 GEMM for bf16 operands at the shapes it serves (N % 128 == 0, K % 64
    == 0), else the device BLAS (other dtypes: fp32 callers of the generic ops)."""
    N, K = w_nk.shape
    if a.dtype == torch.bfloat16 and a.is_cuda and N % 128 == 0 and K % 64 == 0:
        return bf16_gemm(a, w_nk.to(torch.bfloat16), bias=bias, residual=residual)
    out = a @ w_nk.to(a.dtype).t()
    if bias is not None:
        out = out + bias.to(out.dtype)
    if residual is not None:
        out = out + residual.to(out.dtype)
    return out


def scaled_addmm_fp8_preq(activation_fp8: torch.Tensor, scale_a: torch.Tensor, weight: Weight,
                          bias_or_residual: Optional[torch.Tensor], *, out_dtype: torch.dtype = torch.bfloat16,
                          silu_cols: Optional[Tuple[int, int]] = None) -> torch.Tensor:
    """bf16 projection of an e4m3 activation with a 1-D bias or a 2-D residual
    (``scaled_addmm_fp8_preq``, ``triton_fp8.py:1756``).  ``silu_cols`` fuses
    SiLU on a column range (the U slice)."""
    if out_dtype != torch.bfloat16:
        raise ValueError("scaled_addmm_fp8_preq produces bf16")
    bias = residual = None
    if bias_or_residual is not None:
        if bias_or_residual.dim() == 1:
            bias = bias_or_residual
        else:
            residual = bias_or_residual
    return fp8_gemm(activation_fp8, scale_a, weight, bias=bias, residual=residual, silu_cols=silu_cols)


def scaled_mm_fp8_out_preq(activation_fp8: torch.Tensor, scale_a: torch.Tensor, weight: Weight,
                           bias: Optional[torch.Tensor] = None, *,
                           output_scale: Optional[torch.Tensor] = None) -> torch.Tensor:
    """e4m3 projection at ``output_scale`` (``scaled_mm_fp8_out_preq``,
    ``triton_fp8.py:2409``): e4m3(clamp((acc*sa*sw + bias)/output_scale, +-448))."""
    return fp8_gemm(activation_fp8, scale_a, weight, bias=bias, out_dtype=E4M3, out_scale=output_scale)
