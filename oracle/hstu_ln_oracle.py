"""CPU oracle for the output block around the HSTU attention: LayerNorm * U *
dropout with the [u | x | y] concat, its Philox dropout mask, and the weighted
LayerNorm with e4m3 output.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports this file:
only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg use it, and only as the checker.

Reference paths are relative to
``recommendation_v4/hstu/generative_recommenders/``.  Triton (the reference's
third-party kernel language, not vendored) defines ``tl.randint4x`` /
``tl.uint_to_uniform_float``; the reference restates the former itself as
``_philox4x32_10_mad64`` (``ops/triton/triton_hstu_linear.py:289-316``) and the
latter's fp32 test as ``_mask_keep`` / ``_mask_keep_above`` (:319-328,
:2335-2355), and those restatements are what this file follows.

Pinning (checks in ``tests/test_ln_oracle.py``):

* ``philox4x32``        -- the Random123 known-answer vectors of Philox4x32-10
  (Salmon et al., SC'11; kat_vectors of the Random123 distribution).
* ``mask_keep_above``   -- the integer rule against Triton's fp32 test
  ``fp32(fp32(x') * 4.6566127342e-10) > fp32(p)`` on random and boundary x'.
* ``dropout_mask``      -- Philox as above; the row -> (group, word, half)
  layout against an independent restatement of the reference's compact-row
  kernels (``_generate_indexed_random_mask[16]``, :377-426, :473-508), which the
  reference states give "selected rows of a full mask" (:2604); drop rates
  within binomial bounds; p = 0 keeps and p = 1 drops everything.
* ``ln_mul_dropout_fwd`` -- ``torch.nn.functional.layer_norm`` (a library
  routine) for the normalisation, numpy mean / variance for mean / rstd,
  closed forms (u = 1 with no activation gives plain LayerNorm; the concat
  blocks are u / silu(u) and x verbatim; an all-kept mask scales by 1/(1-p),
  an all-dropped one gives zeros).
* ``ln_mul_dropout_bwd`` -- ``torch.autograd`` on the float64 forward and
  ``torch.autograd.gradcheck``.
"""

from __future__ import annotations

from typing import Optional, Tuple

import numpy as np
import torch
import torch.nn.functional as F

_M0 = np.uint64(0xD2511F53)
_M1 = np.uint64(0xCD9E8D57)
_W0 = 0x9E3779B9
_W1 = 0xBB67AE85
_MASK32 = np.uint64(0xFFFFFFFF)
UNIFORM_SCALE = np.float32(4.6566127342e-10)


# --------------------------------------------------------------------------
# Philox4x32-10
# --------------------------------------------------------------------------
def philox4x32(c, k0: int, k1: int, rounds: int = 10):
    """Philox4x32 on counters ``c = (c0, c1, c2, c3)`` (uint32 arrays) with
    key ``(k0, k1)``; returns the four output words as uint32 arrays.
    One round: (hi(M1*c2)^c1^k0, lo(M1*c2), hi(M0*c0)^c3^k1, lo(M0*c0)); the
    key is bumped by the Weyl constants between rounds
    (``triton_hstu_linear.py:301-316``)."""
    c0, c1, c2, c3 = (np.asarray(x, dtype=np.uint64) & _MASK32 for x in c)
    ka, kb = np.uint64(k0 & 0xFFFFFFFF), np.uint64(k1 & 0xFFFFFFFF)
    for _ in range(rounds):
        pa = c0 * _M0
        pb = c2 * _M1
        n0 = (pb >> np.uint64(32)) ^ c1 ^ ka
        n2 = (pa >> np.uint64(32)) ^ c3 ^ kb
        c1 = pb & _MASK32
        c3 = pa & _MASK32
        c0, c2 = n0, n2
        ka = np.uint64((int(ka) + _W0) & 0xFFFFFFFF)
        kb = np.uint64((int(kb) + _W1) & 0xFFFFFFFF)
    return tuple(x.astype(np.uint32) for x in (c0, c1, c2, c3))


def randint4x(seed: int, offsets: np.ndarray):
    """``tl.randint4x(seed, offset)``: counter (offset, 0, 0, 0), key = the
    seed's low and high 32-bit words (``triton_hstu_linear.py:296-300``)."""
    off = np.asarray(offsets, dtype=np.int64).astype(np.uint64) & _MASK32
    z = np.zeros_like(off)
    seed = int(seed) & 0xFFFFFFFFFFFFFFFF
    return philox4x32((off, z, z, z), seed & 0xFFFFFFFF, seed >> 32)


# --------------------------------------------------------------------------
# keep thresholds
# --------------------------------------------------------------------------
def uniform_keep(xp: np.ndarray, p: float) -> np.ndarray:
    """Triton's fp32 dropout test on x' = x ^ (x >> 31):
    fp32(fp32(x') * 4.6566127342e-10) > fp32(p)."""
    v = np.asarray(xp, dtype=np.int64).astype(np.float32) * UNIFORM_SCALE
    return v > np.float32(p)


def mask_keep_above(p: float) -> int:
    """Largest dropped x' in [-1, 2**31 - 1]: binary search of the monotone
    fp32 test (``triton_hstu_linear.py:2335-2355``)."""
    lo, hi = 0, 2 ** 31
    while lo < hi:
        mid = (lo + hi) // 2
        if bool(uniform_keep(np.array([mid]), p)[0]):
            hi = mid
        else:
            lo = mid + 1
    return lo - 1


def mask_keep_min16(p: float) -> int:
    """Smallest kept 16-bit half: round(p * 65536) clamped to [0, 65536]
    (``triton_hstu_linear.py:2542-2544``; Python round, ties to even)."""
    return min(max(int(round(float(p) * 65536.0)), 0), 65536)


def _xprime(words: np.ndarray) -> np.ndarray:
    x = words.astype(np.uint32).view(np.int32).astype(np.int64)
    return x ^ (x >> 31)


# --------------------------------------------------------------------------
# dropout masks
# --------------------------------------------------------------------------
def block_d(D: int) -> int:
    return 1 << max(0, (int(D) - 1).bit_length())


def dropout_mask(N: int, D: int, num_masks: int, p: float, seed: int, mask16: bool) -> np.ndarray:
    """int8 [N, D]; bit j = keep decision of mask j (bit 0 = y, then x, then u).

    32-bit scheme (``_generate_random_mask``, :331-375): rows in groups of 4;
    group g, mask j, column c use counter g*nm*BD + j*BD + c; word i decides
    row 4g+i: keep iff x' > keep_above(p).
    16-bit scheme (``_generate_random_mask16``, :428-470): groups of 8; word
    i's low half decides row 8g+i, its high half row 8g+i+4: keep iff
    half >= keep_min16(p).  Counters are int32 in the reference (wrap mod 2^32).
    """
    BD = block_d(D)
    rows_per = 8 if mask16 else 4
    G = (N + rows_per - 1) // rows_per
    out = np.zeros((G * rows_per, D), dtype=np.int64)
    g = np.arange(G, dtype=np.int64)[:, None]
    c = np.arange(D, dtype=np.int64)[None, :]
    if mask16:
        thr = mask_keep_min16(p)
    else:
        thr = mask_keep_above(p)
    for j in range(num_masks):
        off = (g * (num_masks * BD) + j * BD + c) & 0xFFFFFFFF
        w = randint4x(seed, off)
        for i in range(4):
            if mask16:
                lo = (w[i] & np.uint32(0xFFFF)).astype(np.int64) >= thr
                hi = (w[i] >> np.uint32(16)).astype(np.int64) >= thr
                out[i::8] |= lo.astype(np.int64) << j
                out[i + 4::8] |= hi.astype(np.int64) << j
            else:
                keep = _xprime(w[i]) > thr
                out[i::4] |= keep.astype(np.int64) << j
    return out[:N].astype(np.int8)


def dropout_mask_rows(row_indices, D: int, num_masks: int, p: float, seed: int, mask16: bool) -> np.ndarray:
    """Mask rows of a full-tensor mask picked by their logical row index, the
    way the reference's compact-row kernels compute them: per row, Philox at
    group = row // 4 (or // 8), select word row % 4 (and, for the 16-bit
    scheme, the high half when row % 8 >= 4) (:377-426, :473-508)."""
    BD = block_d(D)
    rows = np.asarray(row_indices, dtype=np.int64)
    out = np.zeros((len(rows), D), dtype=np.int64)
    thr = mask_keep_min16(p) if mask16 else mask_keep_above(p)
    cols = np.arange(D, dtype=np.int64)
    for n, r in enumerate(rows):
        grp, lane = (r // 8, r % 8) if mask16 else (r // 4, r % 4)
        for j in range(num_masks):
            off = (grp * (num_masks * BD) + j * BD + cols) & 0xFFFFFFFF
            w = randint4x(seed, off)[int(lane % 4)]
            if mask16:
                half = (w >> np.uint32(16)) if lane >= 4 else (w & np.uint32(0xFFFF))
                keep = half.astype(np.int64) >= thr
            else:
                keep = _xprime(w) > thr
            out[n] |= keep.astype(np.int64) << j
    return out.astype(np.int8)


def mask_bits(concat_u: bool, concat_x: bool) -> Tuple[int, int]:
    """(u bit, x bit) of the packed mask; 0 = block absent
    (``triton_hstu_linear.py:630-650``)."""
    xb = 2 if concat_x else 0
    ub = (4 if concat_x else 2) if concat_u else 0
    return ub, xb


def dropout_scale(p: float) -> np.float32:
    """fp32(1 / fp32(1 - p)), the kernels' keep scale."""
    return np.float32(np.float32(1.0) / (np.float32(1.0) - np.float32(p)))


# --------------------------------------------------------------------------
# LayerNorm * U * dropout
# --------------------------------------------------------------------------
ACTS = ("none", "silu", "sigmoid")


def ln_mul_dropout_fwd(
    x: torch.Tensor,
    u: Optional[torch.Tensor],
    weight: torch.Tensor,
    bias: torch.Tensor,
    eps: float,
    dropout_ratio: float = 0.0,
    mask: Optional[np.ndarray] = None,
    silu_u: bool = False,
    concat_u: bool = False,
    concat_x: bool = False,
    mul_u_activation_type: str = "none",
    dtype=torch.float64,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(y, mean, rstd) before any output cast.

    y = [u' | x | m(u) * LN(x)] (``pt_hstu_linear.py:23-82``); u' = silu(u)
    when silu_u; m = identity / silu / sigmoid.  With ``mask`` (int8 [N, D],
    training dropout) each block is kept and scaled by 1/(1-p) or zeroed per its
    bit (``triton_hstu_linear.py:620-650``).  ``u = None``: the weighted
    LayerNorm (``ops/triton/triton_layer_norm.py:1668``).
    """
    xf = x.to(dtype)
    D = xf.shape[-1]
    mean = xf.mean(dim=-1)
    var = ((xf - mean[:, None]) ** 2).mean(dim=-1)
    rstd = 1.0 / torch.sqrt(var + eps)
    y = F.layer_norm(xf, (D,), weight.to(dtype), bias.to(dtype), eps)
    blocks = []
    if u is not None:
        uf = u.to(dtype)
        if mul_u_activation_type == "silu":
            m = F.silu(uf)
        elif mul_u_activation_type == "sigmoid":
            m = torch.sigmoid(uf)
        else:
            m = uf
        y = y * m
        if concat_u:
            blocks.append(F.silu(uf) if silu_u else uf)
    if concat_x:
        blocks.append(xf)
    if mask is not None:
        s = float(dropout_scale(dropout_ratio))
        mk = torch.from_numpy(mask.astype(np.int64))
        ub, xb = mask_bits(u is not None and concat_u, concat_x)

        def drop(v, bit):
            return torch.where((mk & bit) != 0, v * s, torch.zeros_like(v))

        y = drop(y, 1)
        kept = []
        if u is not None and concat_u:
            kept.append(drop(blocks[0], ub))
        if concat_x:
            kept.append(drop(blocks[-1], xb))
        blocks = kept
    return torch.cat(blocks + [y], dim=1), mean, rstd


def ln_mul_dropout_bwd(
    dy: torch.Tensor,
    x: torch.Tensor,
    u: Optional[torch.Tensor],
    weight: torch.Tensor,
    bias: torch.Tensor,
    eps: float,
    **kw,
):
    """(dx, du, dweight, dbias) by torch.autograd through
    ``ln_mul_dropout_fwd`` in float64 (the mask is a constant)."""
    xs = x.detach().to(torch.float64).requires_grad_(True)
    us = None if u is None else u.detach().to(torch.float64).requires_grad_(True)
    ws = weight.detach().to(torch.float64).requires_grad_(True)
    bs = bias.detach().to(torch.float64).requires_grad_(True)
    y, _, _ = ln_mul_dropout_fwd(xs, us, ws, bs, eps, dtype=torch.float64, **kw)
    y.backward(dy.to(torch.float64))
    return xs.grad, (None if us is None else us.grad), ws.grad, bs.grad


def e4m3_bytes(v: torch.Tensor, inv_scale: float) -> torch.Tensor:
    """e4m3(clamp(fp32(v) * fp32(inv_scale), +-448)) via torch's RNE cast."""
    f = v.to(torch.float32) * torch.tensor(inv_scale, dtype=torch.float32)
    return f.clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
