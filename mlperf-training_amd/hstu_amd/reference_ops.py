"""The attention custom ops under the reference's own names and schemas.

The reference registers (paths relative to
``recommendation_v4/hstu/generative_recommenders/``):

* ``generative_recommenders::triton_hstu_attention_fwd``
  (``ops/triton/triton_hstu_attention.py:3166-3185``; fake :3490-3524)
* ``generative_recommenders::triton_hstu_attention_bwd``, mutating dq, dk, dv
  (:3298-3319; fake :3527-3547)
* ``generative_recommenders::triton_hstu_attention_delta_bwd``, mutating dq,
  dk, dv (:3413-3428; fake :3483-3497)

Here the same qualified names and argument lists dispatch to this build's
HIP kernels, so code that calls ``torch.ops.generative_recommenders.*`` (or
traces through them) runs unchanged.  The scales are per-tensor floats, as
in the reference's schemas; the per-(token, head) scales and the relative
bias are served by this build's own ``hstu_amd::`` ops.  The forward
allocates its output (bf16 for e4m3 inputs, else v's dtype); the backward
ops write the caller's tensors and zero them for an empty batch.

If the reference's module already registered these names in this process,
its registration is kept and this module registers nothing.
"""

from __future__ import annotations

import logging
from typing import Optional

import torch

from . import hstu_attention as _attn
from . import hstu_delta as _delta

logger = logging.getLogger(__name__)

NAMESPACE = "generative_recommenders"
_E4M3 = getattr(torch, "float8_e4m3fn", None)


def _exists(name: str) -> bool:
    try:
        torch._C._dispatch_find_schema_or_throw(f"{NAMESPACE}::{name}", "")
        return True
    except RuntimeError:
        return False


def _out_dtype(v: torch.Tensor) -> torch.dtype:
    return torch.bfloat16 if (_E4M3 is not None and v.dtype == _E4M3) else v.dtype


def _fwd(N: int, alpha: float, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, seq_offsets: torch.Tensor,
         num_targets: Optional[torch.Tensor], max_attn_len: int, contextual_seq_len: int,
         sort_by_length_indices: Optional[torch.Tensor], enable_tma: bool, num_softmax_heads: int,
         q_scale: float = 1.0, k_scale: float = 1.0, v_scale: float = 1.0) -> torch.Tensor:
    if q.shape[0] == 0:
        return torch.empty((0, q.shape[1], v.shape[2]), dtype=_out_dtype(v), device=v.device)
    out = _attn.triton_hstu_attention_fwd(N, alpha, q, k, v, seq_offsets, num_targets, max_attn_len,
                                          contextual_seq_len, sort_by_length_indices, enable_tma,
                                          num_softmax_heads, q_scale, k_scale, v_scale)
    return out.to(_out_dtype(v))


def _fwd_fake(N, alpha, q, k, v, seq_offsets, num_targets, max_attn_len, contextual_seq_len,
              sort_by_length_indices, enable_tma, num_softmax_heads, q_scale=1.0, k_scale=1.0, v_scale=1.0):
    return torch.empty((q.shape[0], q.shape[1], v.shape[2]), dtype=_out_dtype(v), device=v.device)


def _bwd(dout: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, dq: torch.Tensor,
         dk: torch.Tensor, dv: torch.Tensor, seq_offsets: torch.Tensor, num_targets: Optional[torch.Tensor],
         N: int, alpha: float, max_attn_len: int, contextual_seq_len: int,
         sort_by_length_indices: Optional[torch.Tensor], enable_tma: bool, num_softmax_heads: int) -> None:
    if dout.shape[0] == 0:
        dq.zero_()
        dk.zero_()
        dv.zero_()
        return
    fp8 = _E4M3 is not None and q.dtype == _E4M3
    unit = 1.0 if fp8 else None
    _attn.triton_hstu_attention_bwd(dout, q, k, v, dq, dk, dv, seq_offsets, num_targets, N, alpha, max_attn_len,
                                    contextual_seq_len, sort_by_length_indices, enable_tma, num_softmax_heads,
                                    unit, unit, unit)


def _bwd_fake(dout, q, k, v, dq, dk, dv, seq_offsets, num_targets, N, alpha, max_attn_len, contextual_seq_len,
              sort_by_length_indices, enable_tma, num_softmax_heads) -> None:
    return None


def _delta_bwd(dout: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, dq: torch.Tensor,
               dk: torch.Tensor, dv: torch.Tensor, seq_offsets: torch.Tensor, N: int, alpha: float,
               k_scale: float = 1.0, v_scale: float = 1.0) -> None:
    B = seq_offsets.shape[0] - 1
    if dout.shape[0] != 0 and (q.shape[0] != B or dout.shape[0] != B):
        raise ValueError("delta attention training requires one query per sequence")
    _delta.triton_hstu_attention_delta_bwd(dout, q, k, v, dq, dk, dv, seq_offsets, N, alpha, k_scale, v_scale)


def _delta_bwd_fake(dout, q, k, v, dq, dk, dv, seq_offsets, N, alpha, k_scale=1.0, v_scale=1.0) -> None:
    return None


_OPS = (
    ("triton_hstu_attention_fwd", _fwd, _fwd_fake, ()),
    ("triton_hstu_attention_bwd", _bwd, _bwd_fake, ("dq", "dk", "dv")),
    ("triton_hstu_attention_delta_bwd", _delta_bwd, _delta_bwd_fake, ("dq", "dk", "dv")),
)

registered = {}


def register() -> None:
    """Register the three ops (once per process)."""
    for name, impl, fake, mutates in _OPS:
        if name in registered:
            continue
        if _exists(name):
            logger.warning("[hstu-hip] %s::%s is already registered; keeping it", NAMESPACE, name)
            registered[name] = None
            continue
        op = torch.library.custom_op(f"{NAMESPACE}::{name}", impl, mutates_args=mutates)
        op.register_fake(fake)
        registered[name] = op


register()
