"""The reference's PYTORCH backend of ``hstu_mha`` (selected explicitly with
``kernel=HammerKernel.PYTORCH``, the reference's default), written with plain
torch ops so it runs on whatever device the inputs live on.

Follows ``ops/pytorch/pt_hstu_attention.py:32-187``; the two FBGEMM jagged
ops it calls there are replaced by index arithmetic in torch.  This is a
user-selected backend, never a fallback for the HIP kernels.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F


def _jagged_index(seq_offsets: torch.Tensor, N: int):
    """(batch id, position) for every jagged row, and a keep mask for rows
    whose position is < N."""
    T = int(seq_offsets[-1].item())
    lengths = seq_offsets[1:] - seq_offsets[:-1]
    b = torch.repeat_interleave(torch.arange(lengths.numel(), device=seq_offsets.device), lengths,
                                output_size=T)
    pos = torch.arange(T, device=seq_offsets.device) - seq_offsets[:-1][b]
    return b, pos, pos < N


def jagged_to_padded_dense(values: torch.Tensor, seq_offsets: torch.Tensor, N: int) -> torch.Tensor:
    """[T, F] -> [B, N, F], zero padded (``torch.ops.fbgemm.jagged_to_padded_dense``)."""
    B = seq_offsets.numel() - 1
    b, pos, keep = _jagged_index(seq_offsets, N)
    out = values.new_zeros((B, N) + tuple(values.shape[1:]))
    out[b[keep], pos[keep]] = values[keep]
    return out


def dense_to_jagged(dense: torch.Tensor, seq_offsets: torch.Tensor, T: int) -> torch.Tensor:
    """[B, N, F] -> [T, F]; rows at positions >= N are zero (``dense_to_jagged``)."""
    N = dense.shape[1]
    b, pos, keep = _jagged_index(seq_offsets, N)
    out = dense.new_zeros((T,) + tuple(dense.shape[2:]))
    out[keep] = dense[b[keep], pos[keep]]
    return out


def get_valid_attn_mask(device, causal: bool, N: int, seq_lengths: torch.Tensor,
                        num_targets: Optional[torch.Tensor] = None, max_attn_len: int = 0,
                        contextual_seq_len: int = 0, min_full_attn_seq_len: int = 0) -> torch.Tensor:
    """``_get_valid_attn_mask`` (``pt_hstu_attention.py:32-84``)."""
    ids = torch.arange(0, N, device=device).view(1, N)
    max_ids = seq_lengths.view(-1, 1, 1)
    if contextual_seq_len > 0:
        ids = torch.clamp(ids - contextual_seq_len + 1, min=0)
        max_ids = max_ids - contextual_seq_len + 1
    if num_targets is not None:
        max_ids = max_ids - num_targets.view(-1, 1, 1)
        ids = torch.minimum(ids, max_ids)
        row_ids = ids.view(-1, N, 1).expand(-1, N, N)
        col_ids = ids.view(-1, 1, N).expand(-1, N, N)
    else:
        row_ids = ids.view(N, 1).expand(N, N).reshape(1, N, N)
        col_ids = ids.view(1, N).expand(N, N).reshape(1, N, N)
    dist = row_ids - col_ids
    valid = torch.eye(N, device=device, dtype=torch.bool).view(1, N, N)
    if not causal:
        dist = torch.where(dist > 0, dist, -dist)
    valid = valid | (dist > 0)
    if max_attn_len > 0:
        if min_full_attn_seq_len > 0:
            valid = valid & ((dist <= max_attn_len) | (row_ids >= max_ids - min_full_attn_seq_len))
        else:
            valid = valid & (dist <= max_attn_len)
    if contextual_seq_len > 0:
        valid = valid | ((row_ids == 0) & (col_ids < max_ids))
    return valid


def pytorch_hstu_mha(
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
    *,
    attn_bias: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    L, H, D = q.shape
    V = v.shape[2]
    N = max_seq_len

    def pad(x, width):
        return jagged_to_padded_dense(x.reshape(L, H * width), seq_offsets, N).view(-1, N, H, width).transpose(1, 2)

    qp, kp, vp = pad(q, D), pad(k, D), pad(v, V)
    s = torch.matmul(qp, kp.transpose(-1, -2).contiguous()) * alpha
    if attn_bias is not None:
        R = (attn_bias.shape[1] + 1) // 2
        ar = torch.arange(N, device=q.device)
        idx = torch.clamp(ar.view(N, 1) - ar.view(1, N), -(R - 1), R - 1) + (R - 1)
        s = s + attn_bias[:, idx].unsqueeze(0).to(s.dtype)
    if attn_scale is not None:
        if attn_scale.ndim > 0:
            attn_scale = jagged_to_padded_dense(attn_scale.unsqueeze(-1), seq_offsets, N).unsqueeze(1).to(s.dtype)
        s = F.silu(s) * attn_scale
    else:
        s = F.silu(s) / N
    mask = get_valid_attn_mask(q.device, causal, N, seq_offsets[1:] - seq_offsets[:-1], num_targets,
                               max_attn_len, contextual_seq_len, min_full_attn_seq_len)
    s = s * mask.unsqueeze(1)
    if dropout_pr > 0.0:
        s = F.dropout(s, p=dropout_pr, training=training)
    o = torch.matmul(s, vp)
    return dense_to_jagged(o.transpose(1, 2).flatten(2, 3), seq_offsets, L).view(L, H, V)


def pytorch_cached_hstu_mha(
    max_seq_len: int,
    alpha: float,
    delta_q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    seq_offsets: torch.Tensor,
    num_targets: Optional[torch.Tensor] = None,
    max_attn_len: int = 0,
    contextual_seq_len: int = 0,
) -> torch.Tensor:
    """Delta-q attention (``pt_hstu_attention.py:191-251``): the DS = rows/B
    compact queries of each sequence sit at its last DS positions and use those
    rows of the valid mask against the padded keys."""
    Ld, H, D = delta_q.shape
    V = v.shape[2]
    B = seq_offsets.numel() - 1
    ds = Ld // B
    N = max_seq_len
    qd = delta_q.view(B, ds, H, D).transpose(1, 2)
    kp = jagged_to_padded_dense(k.reshape(-1, H * D), seq_offsets, N).view(B, N, H, D).transpose(1, 2)
    vp = jagged_to_padded_dense(v.reshape(-1, H * V), seq_offsets, N).view(B, N, H, V).transpose(1, 2)
    s = F.silu(torch.matmul(qd, kp.transpose(-1, -2).contiguous()) * alpha) / N
    lengths = seq_offsets[1:] - seq_offsets[:-1]
    full = get_valid_attn_mask(delta_q.device, True, N, lengths, num_targets, max_attn_len,
                               contextual_seq_len).expand(B, N, N)
    pos = torch.arange(N, device=delta_q.device).view(1, -1)
    rows = (pos >= (lengths - ds).view(-1, 1)) & (pos < lengths.view(-1, 1))
    mask = full[rows.view(B, N, 1).expand(B, N, N)].view(B, ds, N)
    s = s * mask.unsqueeze(1)
    return torch.matmul(s, vp).transpose(1, 2).reshape(Ld, H, V)
