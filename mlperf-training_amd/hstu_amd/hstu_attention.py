"""HSTU jagged attention: the reference's Python-visible op surface, served by
this build's gfx950 HIP kernels.

Drop-in names (reference file:line, relative to
``recommendation_v4/hstu/generative_recommenders/``):

* ``hstu_mha``                 <- ``ops/hstu_attention.py:202-329``
* ``triton_hstu_mha``          <- ``ops/triton/triton_hstu_attention.py:3680-3707``
* ``triton_hstu_attention_fwd``<- custom op ``generative_recommenders::triton_hstu_attention_fwd``
                                  (``triton_hstu_attention.py:3166-3295``)
* ``triton_hstu_attention_bwd``<- custom op ``..._bwd`` with ``mutates_args=("dq","dk","dv")``
                                  (``triton_hstu_attention.py:3298-3410``)
* ``try_hstu_attention_fwd`` / ``try_hstu_attention_bwd`` <- the FlyDSL
  ``try_flydsl_attention_fwd`` (-> Optional[Tensor]) / ``try_flydsl_attention_bwd``
  (-> bool) conventions (``ops/flydsl/hstu_flydsl_mha.py:2063-2107, 1787-1869``).

Differences from the reference, all opt-in keyword extras defaulting to the
reference behaviour: ``q_scale``/``k_scale``/``v_scale`` may be per-tensor
floats (as in the reference) or fp32 tensors of shape [T, H] (per token and
head); ``attn_bias`` adds a learned relative-position bias (no reference
counterpart).  Outputs/gradients are bf16.

Host problems raise (``HstuUnavailableError``); an unsupported shape makes the
``try_*`` entry points return None/False with the reason logged once, and makes
the kernel ops raise -- there is no silent fallback to another backend.
"""

from __future__ import annotations

import logging
import os
from enum import Enum, unique
from typing import Optional, Tuple, Union

import torch

from . import _lib

logger = logging.getLogger(__name__)

_E4M3 = getattr(torch, "float8_e4m3fn", None)
ScaleArg = Union[None, float, torch.Tensor]


@unique
class HammerKernel(Enum):
    """Backend selector (``common.py:114-123``).  TRITON and HIP both select
    this build's HIP kernels; PYTORCH selects ``pytorch_hstu_mha``."""

    PYTORCH = "PYTORCH"
    TRITON = "TRITON"
    HIP = "HIP"


# ---------------------------------------------------------------------------
# shape / layout policy
# ---------------------------------------------------------------------------
def _is_fp8(t: torch.Tensor) -> bool:
    return _E4M3 is not None and t.dtype == _E4M3


def unsupported_shape_reason(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    num_softmax_heads: int = 0,
) -> Optional[str]:
    """None when the HIP kernels serve this call, else a reason string
    (the role of ``unsupported_fp8_fwd_shape_reason``,
    ``ops/flydsl/hstu_flydsl_mha.py:311-354``)."""
    if q.dim() != 3 or k.shape != q.shape or v.dim() != 3 or v.shape[:2] != q.shape[:2]:
        return f"shapes q{tuple(q.shape)} k{tuple(k.shape)} v{tuple(v.shape)}"
    if v.shape[2] != q.shape[2]:
        return f"d_v={v.shape[2]} != d_qk={q.shape[2]}"
    if not (q.dtype == k.dtype == v.dtype):
        return f"mixed dtypes {q.dtype}/{k.dtype}/{v.dtype}"
    D = q.shape[2]
    if q.dtype == torch.bfloat16:
        if D not in (64, 128):
            return f"bf16 head dim {D} (kernels are built for 64 and 128)"
    elif _is_fp8(q):
        if D != 128:
            return f"e4m3 head dim {D} (kernel is built for 128)"
    else:
        return f"dtype {q.dtype} (kernels take bf16 or float8_e4m3fn)"
    if num_softmax_heads != 0:
        return "num_softmax_heads != 0"
    if not q.is_cuda:
        return "tensors are not on a GPU"
    return None


def _row_view(t: torch.Tensor) -> torch.Tensor:
    """A view whose element (t, h, d) is at t*stride(0) + h*D + d with
    16-byte aligned rows, so column slices of a fused UVQK buffer are read in
    place (``_common_row_stride``, ``ops/flydsl/hstu_flydsl_mha.py:367-388``);
    anything else is made contiguous."""
    T, H, D = t.shape
    es = t.element_size()
    if (t.stride(2) == 1 and t.stride(1) == D and (T <= 1 or t.stride(0) >= H * D)
            and (t.stride(0) * es) % 16 == 0 and t.data_ptr() % 16 == 0):
        return t
    return t.contiguous()


def _row_stride(t: torch.Tensor) -> int:
    return t.stride(0) if t.shape[0] > 1 else t.shape[1] * t.shape[2]


def _scale_tensor(s: ScaleArg, T: int, H: int, device) -> Tuple[Optional[torch.Tensor], int, int]:
    """(tensor, row_stride, head_stride) for the C ABI's scale addressing."""
    if s is None:
        return None, 0, 0
    if not isinstance(s, torch.Tensor):
        return torch.full((1,), float(s), dtype=torch.float32, device=device), 0, 0
    s = s.to(device=device, dtype=torch.float32)
    if s.numel() == 1:
        return s.reshape(1).contiguous(), 0, 0
    if s.shape != (T, H):
        raise ValueError(f"scale shape {tuple(s.shape)}; expected [T={T}, H={H}] or a scalar")
    s = s.contiguous()
    return s, H, 1


def _workspace(nbytes: int, device) -> torch.Tensor:
    """Caller-owned device workspace of an entry point (the library allocates nothing)."""
    if nbytes < 0:
        raise ValueError("bad sizes for the workspace query")
    return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)


def _seq_offsets_i64(seq_offsets: torch.Tensor) -> torch.Tensor:
    return seq_offsets.to(torch.int64).contiguous()


def _num_targets_i32(num_targets: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    return None if num_targets is None else num_targets.to(torch.int32).contiguous()


def _bias_args(attn_bias: Optional[torch.Tensor], H: int):
    if attn_bias is None:
        return None, 0
    if attn_bias.dim() != 2 or attn_bias.shape[0] != H or attn_bias.shape[1] % 2 != 1:
        raise ValueError(f"attn_bias shape {tuple(attn_bias.shape)}; expected [H, 2R-1]")
    return attn_bias.to(torch.float32).contiguous(), (attn_bias.shape[1] + 1) // 2


def _stream(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


# ---------------------------------------------------------------------------
# raw launches
# ---------------------------------------------------------------------------
def _launch_fwd(N, alpha, q, k, v, seq_offsets, num_targets, max_attn_len, contextual_seq_len,
                q_scale, k_scale, v_scale, attn_bias, pv_scale: float = 0.0) -> torch.Tensor:
    T, H, D = q.shape
    out = torch.empty((T, H, D), dtype=torch.bfloat16, device=q.device)
    if T == 0:
        return out
    fp8 = _is_fp8(q)
    q, k, v = _row_view(q), _row_view(k), _row_view(v)
    if fp8:
        if q_scale is None or k_scale is None or v_scale is None:
            raise ValueError("e4m3 inputs need q_scale, k_scale and v_scale")
        qs, srs, shs = _scale_tensor(q_scale, T, H, q.device)
        ks, srs2, shs2 = _scale_tensor(k_scale, T, H, q.device)
        vs, srs3, shs3 = _scale_tensor(v_scale, T, H, q.device)
        if not (srs == srs2 == srs3 and shs == shs2 == shs3):
            raise ValueError("q/k/v scales must share one layout (all scalars or all [T, H])")
    else:
        qs = ks = vs = None
        srs = shs = 0
        if any(s is not None and not (isinstance(s, (int, float)) and float(s) == 1.0)
               for s in (q_scale, k_scale, v_scale)):
            raise ValueError("q/k/v scales apply to e4m3 inputs only")
    offs = _seq_offsets_i64(seq_offsets)
    nt = _num_targets_i32(num_targets)
    bias, R = _bias_args(attn_bias, H)
    dt = _lib.HSTU_DTYPE_FP8_E4M3 if fp8 else _lib.HSTU_DTYPE_BF16
    B = offs.numel() - 1
    ws = _workspace(_lib.fn("hstu_attn_fwd_workspace_bytes")(dt, T, B, H, D, int(N)), q.device)
    if pv_scale > 0.0:
        if not fp8:
            raise ValueError("the FP8 P.V forward takes e4m3 inputs")
        st = _lib.fn("hstu_attn_fwd_fp8_pv")(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), _row_stride(q), _row_stride(k), _row_stride(v),
            _lib.ptr(qs), _lib.ptr(ks), _lib.ptr(vs), srs, shs,
            offs.data_ptr(), B, H, D, int(N), float(alpha),
            _lib.ptr(nt), int(max_attn_len), int(contextual_seq_len),
            _lib.ptr(bias), R, float(pv_scale),
            out.data_ptr(), H * D, ws.data_ptr(), ws.numel(), T, _stream(q.device))
        _lib.check(st, "hstu_attn_fwd_fp8_pv")
        return out
    st = _lib.fn("hstu_attn_fwd")(
        dt,
        q.data_ptr(), k.data_ptr(), v.data_ptr(), _row_stride(q), _row_stride(k), _row_stride(v),
        _lib.ptr(qs), _lib.ptr(ks), _lib.ptr(vs), srs, shs,
        offs.data_ptr(), offs.numel() - 1, H, D, int(N), float(alpha),
        _lib.ptr(nt), int(max_attn_len), int(contextual_seq_len),
        _lib.ptr(bias), R,
        out.data_ptr(), H * D, ws.data_ptr(), ws.numel(), T, _stream(q.device))
    _lib.check(st, "hstu_attn_fwd")
    return out


def _launch_bwd(dout, q, k, v, dq, dk, dv, seq_offsets, num_targets, N, alpha, max_attn_len,
                contextual_seq_len, q_scale, k_scale, v_scale, attn_bias, dbias) -> None:
    T, H, D = q.shape
    fp8 = _is_fp8(q)
    q, k, v = _row_view(q), _row_view(k), _row_view(v)
    dout = _row_view(dout.to(torch.bfloat16))
    if fp8:
        if q_scale is None or k_scale is None or v_scale is None:
            raise ValueError("e4m3 inputs need q_scale, k_scale and v_scale")
        qs, srs, shs = _scale_tensor(q_scale, T, H, q.device)
        ks, srs2, shs2 = _scale_tensor(k_scale, T, H, q.device)
        vs, srs3, shs3 = _scale_tensor(v_scale, T, H, q.device)
        if not (srs == srs2 == srs3 and shs == shs2 == shs3):
            raise ValueError("q/k/v scales must share one layout (all scalars or all [T, H])")
    else:
        qs = ks = vs = None
        srs = shs = 0
    targets = []
    for g in (dq, dk, dv):
        if g.dtype != torch.bfloat16:
            raise ValueError("gradients are bf16")
        ok = g.stride(2) == 1 and g.stride(1) == D and (T <= 1 or g.stride(0) >= H * D)
        targets.append(g if ok else torch.empty((T, H, D), dtype=torch.bfloat16, device=q.device))
    offs = _seq_offsets_i64(seq_offsets)
    nt = _num_targets_i32(num_targets)
    bias, R = _bias_args(attn_bias, H)
    if dbias is not None:
        if bias is None or dbias.shape != bias.shape or dbias.dtype != torch.float32 or not dbias.is_contiguous():
            raise ValueError("dbias must be a contiguous fp32 tensor shaped like attn_bias")
    dtype_code = _lib.HSTU_DTYPE_FP8_E4M3 if fp8 else _lib.HSTU_DTYPE_BF16
    ws = _workspace(_lib.fn("hstu_attn_bwd_workspace_bytes")(dtype_code, T, offs.numel() - 1, H, D, int(N), R),
                    q.device)
    st = _lib.fn("hstu_attn_bwd")(
        _lib.HSTU_DTYPE_FP8_E4M3 if fp8 else _lib.HSTU_DTYPE_BF16,
        dout.data_ptr(), _row_stride(dout),
        q.data_ptr(), k.data_ptr(), v.data_ptr(), _row_stride(q), _row_stride(k), _row_stride(v),
        _lib.ptr(qs), _lib.ptr(ks), _lib.ptr(vs), srs, shs,
        offs.data_ptr(), offs.numel() - 1, H, D, int(N), float(alpha),
        _lib.ptr(nt), int(max_attn_len), int(contextual_seq_len),
        _lib.ptr(bias), R,
        targets[0].data_ptr(), targets[1].data_ptr(), targets[2].data_ptr(),
        _row_stride(targets[0]), _row_stride(targets[1]), _row_stride(targets[2]),
        _lib.ptr(dbias), ws.data_ptr(), ws.numel(), T, _stream(q.device))
    _lib.check(st, "hstu_attn_bwd")
    for dst, src in zip((dq, dk, dv), targets):
        if dst is not src:
            dst.copy_(src)


def _launch_bwd_fp8(dout8, e8, q, k, v, dq, dk, dv, seq_offsets, N, alpha, q_scale, k_scale, v_scale,
                    attn_bias, dbias, prescale_log2: Tuple[int, int]) -> None:
    """The full-FP8 backward (``hstu_attn_bwd_fp8``) on an e4m3 dO with its
    block scales (``hstu_do_fp8.quantize_do_e4m3_blk``'s output), P and dS
    cast at 2^prescale_log2[0] and 2^prescale_log2[1]."""
    T, H, D = q.shape
    q, k, v = _row_view(q), _row_view(k), _row_view(v)
    if dout8.dtype != _E4M3 or e8.dtype != torch.uint8 or tuple(e8.shape) != (T, H):
        raise ValueError("expected dO8 e4m3 [T, H, D] and E8 uint8 [T, H]")
    dout8 = _row_view(dout8)
    e8 = e8.contiguous()
    qs, srs, shs = _scale_tensor(q_scale, T, H, q.device)
    ks, srs2, shs2 = _scale_tensor(k_scale, T, H, q.device)
    vs, srs3, shs3 = _scale_tensor(v_scale, T, H, q.device)
    if not (srs == srs2 == srs3 and shs == shs2 == shs3):
        raise ValueError("q/k/v scales must share one layout (all scalars or all [T, H])")
    targets = []
    for g in (dq, dk, dv):
        if g.dtype != torch.bfloat16:
            raise ValueError("gradients are bf16")
        ok = (g.stride(2) == 1 and g.stride(1) == D and (T <= 1 or g.stride(0) >= H * D)
              and (g.stride(0) * 2) % 16 == 0 and g.data_ptr() % 16 == 0)
        targets.append(g if ok else torch.empty((T, H, D), dtype=torch.bfloat16, device=q.device))
    offs = _seq_offsets_i64(seq_offsets)
    bias, R = _bias_args(attn_bias, H)
    if dbias is not None:
        if bias is None or dbias.shape != bias.shape or dbias.dtype != torch.float32 or not dbias.is_contiguous():
            raise ValueError("dbias must be a contiguous fp32 tensor shaped like attn_bias")
    B = offs.numel() - 1
    ws = _workspace(_lib.fn("hstu_attn_bwd_fp8_workspace_bytes")(T, B, H, D, int(N), R), q.device)
    st = _lib.fn("hstu_attn_bwd_fp8")(
        dout8.data_ptr(), e8.data_ptr(), _row_stride(dout8),
        q.data_ptr(), k.data_ptr(), v.data_ptr(), _row_stride(q), _row_stride(k), _row_stride(v),
        _lib.ptr(qs), _lib.ptr(ks), _lib.ptr(vs), srs, shs,
        offs.data_ptr(), B, H, D, int(N), float(alpha), int(prescale_log2[0]), int(prescale_log2[1]),
        _lib.ptr(bias), R, targets[0].data_ptr(), targets[1].data_ptr(), targets[2].data_ptr(),
        _row_stride(targets[0]), _row_stride(targets[1]), _row_stride(targets[2]),
        _lib.ptr(dbias), ws.data_ptr(), ws.numel(), T, _stream(q.device))
    _lib.check(st, "hstu_attn_bwd_fp8")
    for dst, src in zip((dq, dk, dv), targets):
        if dst is not src:
            dst.copy_(src)


# FP8 P.V forward switch and scale: the reference's DLRM_HSTU_FP8_FWD_PV and
# DLRM_HSTU_FP8_FWD_PV_SCALE (ops/flydsl/hstu_flydsl_mha.py:2199-2264), read per call.
FP8_FWD_PV_SCALE_DEFAULT = 10.04
FP8_FWD_PV_POW2 = 8.0  # 2^pv_k, pv_k = 3
_FP8_FWD_PV_SCALE_RANGE = (4.0, 32.0)


def fp8_fwd_pv_enabled() -> bool:
    """``DLRM_HSTU_FP8_FWD_PV=1`` (exactly "1"; anything else is off)."""
    return os.environ.get("DLRM_HSTU_FP8_FWD_PV", "0") == "1"


def fp8_fwd_pv_scale() -> float:
    """The static P scale s of the FP8 P.V forward: ``DLRM_HSTU_FP8_FWD_PV_SCALE``
    unset or empty = 10.04; ``pow2`` or ``0`` = 2^3; otherwise a float in
    [4, 32], rounded to 6 decimals.  Anything else raises ValueError (a typo
    must not silently change the cast)."""
    raw = os.environ.get("DLRM_HSTU_FP8_FWD_PV_SCALE", "")
    v = raw.strip().lower()
    if v == "":
        return FP8_FWD_PV_SCALE_DEFAULT
    if v == "pow2":
        return FP8_FWD_PV_POW2
    try:
        x = float(v)
    except ValueError:
        x = float("nan")
    if x == 0.0:
        return FP8_FWD_PV_POW2
    lo, hi = _FP8_FWD_PV_SCALE_RANGE
    if not (lo <= x <= hi):  # also rejects nan / inf
        raise ValueError(f"DLRM_HSTU_FP8_FWD_PV_SCALE={raw!r}: use unset (10.04), 'pow2', '0' or a float in "
                         f"[{lo:g}, {hi:g}]")
    return round(x, 6)


def fp8_pv_fwd_reason(q: torch.Tensor, num_targets, max_attn_len: int, contextual_seq_len: int,
                      N: Optional[int] = None) -> Optional[str]:
    """None when the FP8 P.V forward kernel serves this call (e4m3 inputs,
    D = 128, the causal mask, max_seq_len ``N`` within the kernel's LDS
    table), else why not."""
    if not _is_fp8(q):
        return "inputs are not e4m3"
    if q.shape[2] != 128:
        return f"head dim {q.shape[2]}"
    if num_targets is not None or max_attn_len > 0 or contextual_seq_len > 0:
        return "num_targets / max_attn_len / contextual_seq_len masks"
    if N is not None:
        n_max = int(_lib.fn("hstu_attn_fwd_fp8_pv_max_seq_len")())
        if int(N) > n_max:
            return f"max_seq_len {int(N)} above {n_max} (the kernel's per-key LDS table)"
    return None


def full_fp8_bwd_reason(q: torch.Tensor, num_targets, max_attn_len: int, contextual_seq_len: int) -> Optional[str]:
    """None when the full-FP8 backward kernels serve this call (e4m3 inputs,
    D = 128, the causal mask), else why not."""
    if not _is_fp8(q):
        return "inputs are not e4m3"
    if q.shape[2] != 128:
        return f"head dim {q.shape[2]}"
    if num_targets is not None or max_attn_len > 0 or contextual_seq_len > 0:
        return "num_targets / max_attn_len / contextual_seq_len masks"
    return None


# ---------------------------------------------------------------------------
# custom ops (same argument lists and mutation contract as the reference)
# ---------------------------------------------------------------------------
@torch.library.custom_op("hstu_amd::hstu_attention_fwd", mutates_args=())
def _op_fwd(
    N: int,
    alpha: float,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    seq_offsets: torch.Tensor,
    num_targets: Optional[torch.Tensor],
    max_attn_len: int,
    contextual_seq_len: int,
    q_scale: Optional[torch.Tensor],
    k_scale: Optional[torch.Tensor],
    v_scale: Optional[torch.Tensor],
    attn_bias: Optional[torch.Tensor],
    pv_scale: float = 0.0,
) -> torch.Tensor:
    return _launch_fwd(N, alpha, q, k, v, seq_offsets, num_targets, max_attn_len, contextual_seq_len,
                       q_scale, k_scale, v_scale, attn_bias, pv_scale)


@_op_fwd.register_fake
def _op_fwd_fake(N, alpha, q, k, v, seq_offsets, num_targets, max_attn_len, contextual_seq_len,
                 q_scale, k_scale, v_scale, attn_bias, pv_scale=0.0):
    return q.new_empty((q.shape[0], q.shape[1], v.shape[2]), dtype=torch.bfloat16)


@torch.library.custom_op("hstu_amd::hstu_attention_bwd", mutates_args=("dq", "dk", "dv", "dbias"))
def _op_bwd(
    dout: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    dq: torch.Tensor,
    dk: torch.Tensor,
    dv: torch.Tensor,
    seq_offsets: torch.Tensor,
    num_targets: Optional[torch.Tensor],
    N: int,
    alpha: float,
    max_attn_len: int,
    contextual_seq_len: int,
    q_scale: Optional[torch.Tensor],
    k_scale: Optional[torch.Tensor],
    v_scale: Optional[torch.Tensor],
    attn_bias: Optional[torch.Tensor],
    dbias: Optional[torch.Tensor],
    full_fp8: bool = False,
    p8_log2: int = 0,
    ds8_log2: int = 0,
) -> None:
    if dout.shape[0] == 0:
        dq.zero_()
        dk.zero_()
        dv.zero_()
        if dbias is not None:
            dbias.zero_()
        return
    if full_fp8:
        from . import hstu_do_fp8

        # the reference's full-FP8 backward: dO quantized in pow2 blocks, then five e4m3 products
        dout8, e8 = hstu_do_fp8.quantize_do_e4m3_blk(dout, seq_offsets, int(N))
        _launch_bwd_fp8(dout8, e8, q, k, v, dq, dk, dv, seq_offsets, N, alpha, q_scale, k_scale, v_scale,
                        attn_bias, dbias, (p8_log2, ds8_log2))
        return
    _launch_bwd(dout, q, k, v, dq, dk, dv, seq_offsets, num_targets, N, alpha, max_attn_len,
                contextual_seq_len, q_scale, k_scale, v_scale, attn_bias, dbias)


@_op_bwd.register_fake
def _op_bwd_fake(dout, q, k, v, dq, dk, dv, seq_offsets, num_targets, N, alpha, max_attn_len,
                 contextual_seq_len, q_scale, k_scale, v_scale, attn_bias, dbias, full_fp8=False, p8_log2=0,
                 ds8_log2=0):
    return None


def _scale_or_none(s: ScaleArg, like: torch.Tensor) -> Optional[torch.Tensor]:
    if s is None:
        return None
    if isinstance(s, torch.Tensor):
        return s
    return torch.full((1,), float(s), dtype=torch.float32, device=like.device)


def triton_hstu_attention_fwd(
    N: int,
    alpha: float,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    seq_offsets: torch.Tensor,
    num_targets: Optional[torch.Tensor],
    max_attn_len: int,
    contextual_seq_len: int,
    sort_by_length_indices: Optional[torch.Tensor],
    enable_tma: bool,
    num_softmax_heads: int,
    q_scale: ScaleArg = 1.0,
    k_scale: ScaleArg = 1.0,
    v_scale: ScaleArg = 1.0,
    *,
    attn_bias: Optional[torch.Tensor] = None,
    fp8_pv: Optional[bool] = None,
) -> torch.Tensor:
    """Forward op with the reference's argument list
    (``triton_hstu_attention.py:3166-3185``).  Allocates and returns the
    [T, H, D] bf16 output.  ``sort_by_length_indices`` and ``enable_tma`` are
    scheduling hints of the reference kernel and do not change results: the HIP
    grid already issues the longest blocks first.

    ``fp8_pv`` (None: ``DLRM_HSTU_FP8_FWD_PV``): for e4m3 inputs, the
    reference's FP8 P.V forward -- the SiLU output rounded to e4m3 with the
    static scale of ``DLRM_HSTU_FP8_FWD_PV_SCALE`` and P.V on the e4m3 MFMA
    (``hstu_attn_fwd_fp8_pv``), a declared precision change.  A call it does
    not serve (the targets / window / contextual masks) runs the bf16-P
    forward, with the reason logged once, as the reference declines."""
    del sort_by_length_indices, enable_tma
    reason = unsupported_shape_reason(q, k, v, num_softmax_heads)
    if reason is not None:
        raise NotImplementedError(f"HIP HSTU attention forward: {reason}")
    fp8 = _is_fp8(q)
    pv_scale = 0.0
    if fp8 and (fp8_fwd_pv_enabled() if fp8_pv is None else fp8_pv):
        why = fp8_pv_fwd_reason(q, num_targets, int(max_attn_len), int(contextual_seq_len), int(N))
        if why is None:
            pv_scale = fp8_fwd_pv_scale()
        else:
            _log_once(f"FP8 P.V forward: {why}; the bf16-P forward runs")
    return _op_fwd(int(N), float(alpha), q, k, v, seq_offsets, num_targets, int(max_attn_len),
                   int(contextual_seq_len),
                   _scale_or_none(q_scale, q) if fp8 else None,
                   _scale_or_none(k_scale, q) if fp8 else None,
                   _scale_or_none(v_scale, q) if fp8 else None,
                   attn_bias, pv_scale)


def triton_hstu_attention_bwd(
    dout: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    dq: torch.Tensor,
    dk: torch.Tensor,
    dv: torch.Tensor,
    seq_offsets: torch.Tensor,
    num_targets: Optional[torch.Tensor],
    N: int,
    alpha: float,
    max_attn_len: int,
    contextual_seq_len: int,
    sort_by_length_indices: Optional[torch.Tensor],
    enable_tma: bool,
    num_softmax_heads: int,
    q_scale: ScaleArg = None,
    k_scale: ScaleArg = None,
    v_scale: ScaleArg = None,
    *,
    attn_bias: Optional[torch.Tensor] = None,
    dbias: Optional[torch.Tensor] = None,
    full_fp8: Optional[bool] = None,
    ssc_k: Optional[int] = None,
    dsc_k: Optional[int] = None,
) -> None:
    """Backward op (``triton_hstu_attention.py:3298-3319``): writes dq, dk, dv
    in place (they may be strided views of a fused gradient buffer); an empty
    batch zeroes them.  With ``attn_bias``, ``dbias`` (fp32, same shape, if
    given) is overwritten with the bias gradient.

    ``full_fp8`` (None: the process default, ``DLRM_HSTU_FP8_BWD_FULL``): for
    e4m3 inputs, the reference's full-FP8 backward -- dO quantized to e4m3 in
    power-of-two (sequence, head, 32-token) blocks, P and dS cast to e4m3,
    all five products on the e4m3 MFMA (``hstu_attn_bwd_fp8``).  A call it
    cannot serve (the targets / window / contextual masks) runs the e4m3-input
    backward on the block-quantized dO instead, with the reason logged once.
    ``ssc_k`` / ``dsc_k``: the P and dS pre-scale exponents relative to
    ceil(log2 N) (None: the reference's environment, read per call,
    ``hstu_do_fp8.full_fp8_prescale_log2``)."""
    del sort_by_length_indices, enable_tma
    reason = unsupported_shape_reason(q, k, v, num_softmax_heads)
    if reason is not None:
        raise NotImplementedError(f"HIP HSTU attention backward: {reason}")
    fp8 = _is_fp8(q)
    use_full = False
    prescale = (0, 0)
    if fp8 and dout.numel() > 0:
        from . import hstu_do_fp8

        if hstu_do_fp8.bwd_full_fp8_enabled() if full_fp8 is None else full_fp8:
            why = full_fp8_bwd_reason(q, num_targets, int(max_attn_len), int(contextual_seq_len))
            H, D = dout.shape[1], dout.shape[2]
            if why is None:
                use_full = True
                prescale = hstu_do_fp8.full_fp8_prescale_log2(int(N), ssc_k=ssc_k, dsc_k=dsc_k)
            elif D in (64, 128) and H * D in (128, 256, 512):
                _log_once(f"full-FP8 backward: {why}; the e4m3 backward runs on the block-quantized dO")
                dout = hstu_do_fp8.block_quantized_do(dout, seq_offsets, int(N))
            else:
                _log_once(f"full-FP8 backward: {why}; dO quantizer: H*D = {H * D} not served, bf16 dO kept")
    _op_bwd(dout, q, k, v, dq, dk, dv, seq_offsets, num_targets, int(N), float(alpha), int(max_attn_len),
            int(contextual_seq_len),
            _scale_or_none(q_scale, q) if fp8 else None,
            _scale_or_none(k_scale, q) if fp8 else None,
            _scale_or_none(v_scale, q) if fp8 else None,
            attn_bias, dbias, use_full, prescale[0], prescale[1])


# ---------------------------------------------------------------------------
# fallible entry points (FlyDSL try_* conventions)
# ---------------------------------------------------------------------------
_logged_reasons = set()


def _log_once(reason: str) -> None:
    if reason not in _logged_reasons:
        _logged_reasons.add(reason)
        logger.warning("[hstu-hip] declining: %s", reason)


def try_hstu_attention_fwd(
    *, q, k, v, seq_offsets, num_targets, N, alpha, max_attn_len, contextual_seq_len,
    num_softmax_heads=0, q_scale: ScaleArg = None, k_scale: ScaleArg = None, v_scale: ScaleArg = None,
    attn_bias=None, fp8_pv: Optional[bool] = None,
) -> Optional[torch.Tensor]:
    """The HIP forward, or None (reason logged once) when the shape is outside
    the kernels' specialisation.  Host problems raise."""
    reason = unsupported_shape_reason(q, k, v, num_softmax_heads)
    if reason is not None:
        _log_once(reason)
        return None
    return triton_hstu_attention_fwd(N, alpha, q, k, v, seq_offsets, num_targets, max_attn_len,
                                     contextual_seq_len, None, False, num_softmax_heads,
                                     q_scale, k_scale, v_scale, attn_bias=attn_bias, fp8_pv=fp8_pv)


def try_hstu_attention_bwd(
    *, dout, q, k, v, dq, dk, dv, seq_offsets, num_targets, N, alpha, max_attn_len,
    contextual_seq_len, num_softmax_heads=0, q_scale: ScaleArg = None, k_scale: ScaleArg = None,
    v_scale: ScaleArg = None, attn_bias=None,
) -> bool:
    """Writes dq/dk/dv and returns True, or returns False with the outputs
    untouched when the shape is unsupported."""
    reason = unsupported_shape_reason(q, k, v, num_softmax_heads)
    if reason is not None:
        _log_once(reason)
        return False
    triton_hstu_attention_bwd(dout, q, k, v, dq, dk, dv, seq_offsets, num_targets, N, alpha, max_attn_len,
                              contextual_seq_len, None, False, num_softmax_heads, q_scale, k_scale, v_scale,
                              attn_bias=attn_bias)
    return True


# ---------------------------------------------------------------------------
# autograd + public callables
# ---------------------------------------------------------------------------
class _AttentionFunction(torch.autograd.Function):
    """Autograd wrapper (``triton_hstu_attention.py:3563-3677``)."""

    @staticmethod
    def forward(ctx, N, alpha, q, k, v, seq_offsets, num_targets, max_attn_len, contextual_seq_len,
                sort_by_length, enable_tma, attn_bias):
        saved = [q, k, v, seq_offsets]
        if num_targets is not None:
            saved.append(num_targets)
        if attn_bias is not None:
            saved.append(attn_bias)
        ctx.save_for_backward(*saved)
        ctx.has_targets = num_targets is not None
        ctx.has_bias = attn_bias is not None
        ctx.N, ctx.alpha = N, alpha
        ctx.max_attn_len, ctx.contextual_seq_len = max_attn_len, contextual_seq_len
        return triton_hstu_attention_fwd(N, alpha, q, k, v, seq_offsets, num_targets, max_attn_len,
                                         contextual_seq_len, None, enable_tma, 0, attn_bias=attn_bias)

    @staticmethod
    def backward(ctx, dout):
        q, k, v, seq_offsets = ctx.saved_tensors[:4]
        idx = 4
        num_targets = None
        if ctx.has_targets:
            num_targets = ctx.saved_tensors[idx]
            idx += 1
        attn_bias = ctx.saved_tensors[idx] if ctx.has_bias else None
        with torch.inference_mode():
            dq = torch.empty_like(q)
            dk = torch.empty_like(k)
            dv = torch.empty_like(v)
            dbias = None
            if attn_bias is not None:
                dbias = torch.empty(attn_bias.shape, dtype=torch.float32, device=q.device)
            triton_hstu_attention_bwd(dout, q, k, v, dq, dk, dv, seq_offsets, num_targets, ctx.N,
                                      ctx.alpha, ctx.max_attn_len, ctx.contextual_seq_len, None, False, 0,
                                      attn_bias=attn_bias, dbias=dbias)
        return (None, None, dq, dk, dv, None, None, None, None, None, None,
                None if dbias is None else dbias.to(attn_bias.dtype))


def triton_hstu_mha(
    N: int,
    alpha: float,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    seq_offsets: torch.Tensor,
    num_targets: Optional[torch.Tensor] = None,
    max_attn_len: int = 0,
    contextual_seq_len: int = 0,
    sort_by_length: bool = False,
    enable_tma: bool = False,
    *,
    attn_bias: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Differentiable jagged HSTU attention on the HIP kernels
    (signature of ``triton_hstu_mha``, ``triton_hstu_attention.py:3680-3707``)."""
    return _AttentionFunction.apply(N, alpha, q, k, v, seq_offsets, num_targets, max_attn_len,
                                    contextual_seq_len, sort_by_length, enable_tma, attn_bias)


def hstu_mha(
    max_seq_len: int,
    alpha: float,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    seq_offsets: torch.Tensor,
    causal: bool = True,
    dropout_pr: float = 0.0,
    training: bool = True,
    num_targets: Optional[torch.Tensor] = None,
    attn_scale: Optional[torch.Tensor] = None,
    max_attn_len: int = 0,
    contextual_seq_len: int = 0,
    min_full_attn_seq_len: int = 0,
    sort_by_length: bool = False,
    kernel: HammerKernel = HammerKernel.PYTORCH,
    enable_tma: bool = False,
    *,
    attn_bias: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Dispatch with the reference's checks (``ops/hstu_attention.py:202-329``)."""
    H = q.shape[1]
    torch._assert(max_seq_len > 0, "max_seq_len must be larger than 0")
    torch._assert(q.dim() == 3, "q must be 3-D")
    torch._assert(k.shape == q.shape, "k must be the same shape as q")
    torch._assert(v.dim() == 3, "v must be 3-D")
    torch._assert(v.shape[0] == q.shape[0], "wrong v shape[0]")
    torch._assert(v.shape[1] == H, "wrong v shape[1]")
    torch._assert(causal, "only support causal attention")
    if kernel in (HammerKernel.TRITON, HammerKernel.HIP):
        torch._assert(q.is_cuda, "q must be CUDA tensor")
        torch._assert(seq_offsets.is_cuda, "seq_offsets must be CUDA tensor")
        torch._assert(dropout_pr < 1e-6, "dropout for triton path not implemented")
        torch._assert(min_full_attn_seq_len == 0, "min_full_attn_seq_len not implemented")
        assert attn_scale is None, "attn_scale not implemented"
        return triton_hstu_mha(max_seq_len, alpha, q, k, v, seq_offsets, num_targets, max_attn_len,
                               contextual_seq_len, sort_by_length, enable_tma, attn_bias=attn_bias)
    from .pt_hstu_attention import pytorch_hstu_mha

    return pytorch_hstu_mha(max_seq_len, alpha, q, k, v, seq_offsets, causal=True, dropout_pr=dropout_pr,
                            training=training, num_targets=num_targets, attn_scale=attn_scale,
                            max_attn_len=max_attn_len, contextual_seq_len=contextual_seq_len,
                            min_full_attn_seq_len=min_full_attn_seq_len, attn_bias=attn_bias)
