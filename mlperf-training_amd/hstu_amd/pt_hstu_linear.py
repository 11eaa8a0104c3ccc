"""The reference's PYTORCH backend of the HSTU output block (selected
explicitly with ``kernel=HammerKernel.PYTORCH``), in plain torch ops.

Follows ``ops/pytorch/pt_hstu_linear.py:23-120`` (layer-norm variant; group
norm is not served).  This is a user-selected backend, never a fallback for
the HIP kernels.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def pytorch_norm_mul_dropout(
    x: torch.Tensor,
    u: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor,
    eps: float,
    dropout_ratio: float,
    training: bool,
    silu_u: bool = False,
    concat_u: bool = False,
    concat_x: bool = False,
    mul_u_activation_type: str = "none",
    group_norm: bool = False,
    num_heads: int = 1,
    linear_dim: int = -1,
) -> torch.Tensor:
    """dropout([u' | x | m(u) * LN(x)]) in fp32, cast back to x's dtype."""
    if group_norm:
        raise NotImplementedError("group norm is not served by this build")
    dtype = x.dtype
    xf = x.to(torch.float32)
    uf = u.to(torch.float32)
    if mul_u_activation_type == "sigmoid":
        m = torch.sigmoid(uf)
    elif mul_u_activation_type == "silu":
        m = F.silu(uf)
    else:
        m = uf
    y = m * F.layer_norm(xf, (xf.shape[-1],), weight.to(torch.float32), bias.to(torch.float32), eps)
    parts = []
    if concat_u:
        parts.append(F.silu(uf) if silu_u else uf)
    if concat_x:
        parts.append(xf)
    if parts:
        y = torch.cat(parts + [y], dim=1)
    return F.dropout(y, p=dropout_ratio, training=training).to(dtype)


def pytorch_hstu_compute_output(
    attn: torch.Tensor,
    u: torch.Tensor,
    x: torch.Tensor,
    norm_weight: torch.Tensor,
    norm_bias: torch.Tensor,
    output_weight: torch.Tensor,
    eps: float,
    dropout_ratio: float,
    training: bool,
    silu_u: bool = False,
    concat_u: bool = False,
    concat_x: bool = False,
    mul_u_activation_type: str = "none",
    group_norm: bool = False,
    num_heads: int = 1,
    linear_dim: int = -1,
) -> torch.Tensor:
    """x + norm_mul_dropout(attn, u) @ output_weight."""
    y = pytorch_norm_mul_dropout(attn, u, norm_weight, norm_bias, eps, dropout_ratio, training, silu_u,
                                 concat_u, concat_x, mul_u_activation_type, group_norm, num_heads, linear_dim)
    return torch.addmm(x, y, output_weight.to(x.dtype)).to(x.dtype)
