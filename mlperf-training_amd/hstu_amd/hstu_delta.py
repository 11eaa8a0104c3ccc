"""Delta-q ("cached" / targets-only) HSTU attention on this build's kernels
(``hstu_delta_attn_fwd`` / ``hstu_delta_attn_bwd``).

Drop-in names (reference file:line, relative to
``recommendation_v4/hstu/generative_recommenders/``):

* ``triton_cached_hstu_mha``          <- ``ops/triton/triton_hstu_attention.py:3710-3866``
* ``triton_hstu_attention_delta_bwd`` <- custom op with ``mutates_args=("dq", "dk", "dv")``
                                         (``triton_hstu_attention.py:3413-3480``)
* ``delta_hstu_mha``                  <- ``ops/hstu_attention.py:332-420``; the TRITON/HIP
  path is differentiable here (forward + the delta backward), the PYTORCH
  path is ``pytorch_cached_hstu_mha``.

Each sequence's DS = delta_q.shape[0] / B compact query rows are its last DS
positions.  k / v may be e4m3 with per-tensor scales (floats, as the
reference passes them); the output and the gradients are bf16.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from .hstu_attention import HammerKernel
from .pt_hstu_attention import pytorch_cached_hstu_mha

_E4M3 = torch.float8_e4m3fn


def _dt(t: torch.Tensor) -> int:
    if t.dtype == _E4M3:
        return _lib.HSTU_DTYPE_FP8_E4M3
    if t.dtype == torch.bfloat16:
        return _lib.HSTU_DTYPE_BF16
    raise NotImplementedError(f"delta attention serves bf16 / e4m3, not {t.dtype}")


def _rs(t: torch.Tensor) -> int:
    if t.dim() != 3 or t.stride(2) != 1 or t.stride(1) != t.shape[2]:
        raise ValueError("expected [rows, H, D] with contiguous heads (row stride may be wider)")
    return t.stride(0)


def _vec16(t: torch.Tensor) -> torch.Tensor:
    """The kernels read q / dO rows as 16-byte pieces: a small query-side
    tensor whose base or row stride is not 16-byte aligned is copied."""
    if t.data_ptr() % 16 or (t.stride(0) * t.element_size()) % 16:
        return t.clone(memory_format=torch.contiguous_format)
    return t


def _i64(offs: torch.Tensor) -> torch.Tensor:
    return offs.to(torch.int64).contiguous()


def _nt(num_targets: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    return None if num_targets is None else num_targets.to(torch.int32).contiguous()


def _ws(B: int, H: int, D: int, N: int, ds: int, device) -> torch.Tensor:
    n = int(_lib.fn("hstu_delta_attn_workspace_bytes")(B, H, D, N, ds))
    if n < 0:
        raise ValueError("bad sizes for the delta attention workspace")
    return torch.empty((max(n, 4),), dtype=torch.uint8, device=device)


def _kv_dtype(k: torch.Tensor, v: torch.Tensor) -> int:
    dk, dv = _dt(k), _dt(v)
    if dk != dv:
        raise NotImplementedError("k and v must share a dtype")
    return dk


def triton_cached_hstu_mha(
    N: int,
    alpha: float,
    delta_q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    seq_offsets: torch.Tensor,
    num_targets: Optional[torch.Tensor] = None,
    max_attn_len: int = 0,
    contextual_seq_len: int = 0,
    enable_tma: bool = False,
    q_scale: float = 1.0,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
) -> torch.Tensor:
    """[rows, H, D] bf16 output of the delta rows."""
    Ld, H, D = delta_q.shape
    B = seq_offsets.numel() - 1
    if B > 0 and Ld % B:
        raise ValueError("delta_q must hold the same number of rows for every sequence")
    ds = Ld // B if B > 0 else 1
    out = torch.empty((Ld, H, v.shape[2]), dtype=torch.bfloat16, device=delta_q.device)
    if Ld == 0:
        return out
    offs = _i64(seq_offsets)
    nt = _nt(num_targets)
    delta_q = _vec16(delta_q)
    ws = _ws(B, H, D, N, ds, delta_q.device)
    st = _lib.fn("hstu_delta_attn_fwd")(
        _kv_dtype(k, v), _dt(delta_q), delta_q.data_ptr(), k.data_ptr(), v.data_ptr(), _rs(delta_q), _rs(k), _rs(v),
        float(q_scale), float(k_scale), float(v_scale), offs.data_ptr(), B, H, D, N, ds, float(alpha), _lib.ptr(nt),
        int(max_attn_len), int(contextual_seq_len), out.data_ptr(), out.stride(0), ws.data_ptr(), ws.numel(),
        torch.cuda.current_stream(delta_q.device).cuda_stream)
    _lib.check(st, "hstu_delta_attn_fwd")
    return out


def triton_hstu_attention_delta_bwd(
    dout: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    dq: torch.Tensor,
    dk: torch.Tensor,
    dv: torch.Tensor,
    seq_offsets: torch.Tensor,
    N: int,
    alpha: float,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
    *,
    q_scale: float = 1.0,
    num_targets: Optional[torch.Tensor] = None,
    max_attn_len: int = 0,
    contextual_seq_len: int = 0,
) -> None:
    """Writes dq [rows, H, D] and dk, dv [T, H, D] (bf16, caller-owned)."""
    Ld, H, D = q.shape
    B = seq_offsets.numel() - 1
    if Ld == 0 or dout.shape[0] == 0:
        dq.zero_()
        dk.zero_()
        dv.zero_()
        return
    if Ld % B:
        raise ValueError("delta attention training requires the same number of query rows per sequence")
    ds = Ld // B
    for name, t in (("dq", dq), ("dk", dk), ("dv", dv), ("dout", dout)):
        if t.dtype != torch.bfloat16:
            raise ValueError(f"{name} must be bf16")
    offs = _i64(seq_offsets)
    nt = _nt(num_targets)
    q, dout = _vec16(q), _vec16(dout)
    ws = _ws(B, H, D, N, ds, q.device)
    st = _lib.fn("hstu_delta_attn_bwd")(
        _kv_dtype(k, v), _dt(q), dout.data_ptr(), _rs(dout), q.data_ptr(), k.data_ptr(), v.data_ptr(), _rs(q),
        _rs(k), _rs(v), float(q_scale), float(k_scale), float(v_scale), offs.data_ptr(), B, H, D, N, ds,
        float(alpha), _lib.ptr(nt), int(max_attn_len), int(contextual_seq_len), dq.data_ptr(), dk.data_ptr(),
        dv.data_ptr(), _rs(dq), _rs(dk), _rs(dv), ws.data_ptr(), ws.numel(),
        torch.cuda.current_stream(q.device).cuda_stream)
    _lib.check(st, "hstu_delta_attn_bwd")


class _DeltaAttentionFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, N, alpha, delta_q, k, v, seq_offsets, num_targets, max_attn_len, contextual_seq_len):
        ctx.save_for_backward(delta_q, k, v, seq_offsets, *([] if num_targets is None else [num_targets]))
        ctx.cfg = (N, alpha, max_attn_len, contextual_seq_len, num_targets is not None)
        return triton_cached_hstu_mha(N, alpha, delta_q, k, v, seq_offsets, num_targets, max_attn_len,
                                      contextual_seq_len)

    @staticmethod
    def backward(ctx, dout):
        N, alpha, max_attn_len, ctx_len, has_nt = ctx.cfg
        q, k, v, offs = ctx.saved_tensors[:4]
        nt = ctx.saved_tensors[4] if has_nt else None
        dq = torch.empty(q.shape, dtype=torch.bfloat16, device=q.device)
        dk = torch.empty(k.shape, dtype=torch.bfloat16, device=k.device)
        dv = torch.empty(v.shape, dtype=torch.bfloat16, device=v.device)
        triton_hstu_attention_delta_bwd(dout.contiguous(), q, k, v, dq, dk, dv, offs, N, alpha, num_targets=nt,
                                        max_attn_len=max_attn_len, contextual_seq_len=ctx_len)
        return None, None, dq, dk, dv, None, None, None, None


def delta_hstu_mha(
    max_seq_len: int,
    alpha: float,
    delta_q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    seq_offsets: torch.Tensor,
    num_targets: Optional[torch.Tensor] = None,
    max_attn_len: int = 0,
    contextual_seq_len: int = 0,
    kernel: HammerKernel = HammerKernel.PYTORCH,
    enable_tma: bool = False,
) -> torch.Tensor:
    """Delta-q attention (``ops/hstu_attention.py:332-420``)."""
    L, H, D = delta_q.shape
    B = seq_offsets.size(0) - 1
    if max_seq_len <= 0 or delta_q.dim() != 3 or (B > 0 and L % B) or k.shape[1:] != (H, D) or v.shape[1] != H:
        raise ValueError("bad delta attention shapes")
    if kernel in (HammerKernel.TRITON, HammerKernel.HIP):
        return _DeltaAttentionFunction.apply(max_seq_len, alpha, delta_q, k, v, seq_offsets, num_targets,
                                             max_attn_len, contextual_seq_len)
    return pytorch_cached_hstu_mha(max_seq_len, alpha, delta_q, k, v, seq_offsets, num_targets, max_attn_len,
                                   contextual_seq_len)
