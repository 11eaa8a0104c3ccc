"""CPU restatement of the full-FP8 backward's dO block quantizer.

TEST INFRASTRUCTURE ONLY (imported by ``tests/`` and nowhere in the product).

Follows ``ops/flydsl/hstu_do_fp8.py`` (reference paths relative to
``recommendation_v4/hstu/generative_recommenders/``):

* ``group_of``              -- the token grouping G(p) = (p // 64, (p % 16) // 8)
  of the contract text (:16-27).  Pinned by enumeration: every 64-token tile
  splits into two groups of 32, and G is constant on each 8-token run.
* ``group_exp``             -- ``_grp_exp`` (:30-38): floor(log2(448 / amax))
  from the fp32 bits, clamped to [-60, 60], 60 for a subnormal amax, 0 for 0.
  Pinned against ``group_exp_brute`` (the largest integer e with
  amax * 2^e <= 448, found by exact float64 search) on random, power-of-two,
  1.75 * 2^k boundary and neighbouring values, and by the (224, 448] range
  of amax * 2^e.
* ``quantize_do_e4m3_blk``  -- ``_blk_kernel`` / ``quantize_do_e4m3_blk``
  (:42-86, :95-121): per (sequence, head, group) amax, e, dO8 =
  e4m3(dO * 2^e) (torch's RNE float8_e4m3fn conversion, a library routine),
  E8 = 127 - e.  Pinned by the pieces above, the exact decode
  dO8 * 2^-e within half an e4m3 step of dO, and brute-force group maxima.
* ``dequantize_do_e4m3_blk`` -- the undoing of the block scales
  (``hstu_flydsl_mha.py:1330-1394``, inside the reference's MFMAs):
  bf16(dO8 * 2^(E8 - 127)).  Pinned by exactness (the float64 product is a
  bf16 value) and by the round trip staying within half an e4m3 step.
"""

from __future__ import annotations

import numpy as np
import torch

E4M3_MAX = 448.0
TILE = 64


def group_of(p: np.ndarray) -> tuple:
    """(tile, half) of sequence-relative token index p."""
    p = np.asarray(p)
    return p // TILE, (p % 16) // 8


def group_exp(amax: np.ndarray) -> np.ndarray:
    """Bit-level exponent of ``_grp_exp`` for float32 amax >= 0."""
    a = np.asarray(amax, dtype=np.float32)
    bits = a.view(np.int32)
    E = (bits >> 23) & 0xFF
    mant = bits & 0x7FFFFF
    e = np.where(mant <= 0x600000, 135 - E, 134 - E)
    e = np.clip(e, -60, 60)
    e = np.where(E == 0, 60, e)
    return np.where(a == 0.0, 0, e).astype(np.int32)


def group_exp_brute(amax: float) -> int:
    """Largest integer e in [-60, 60] with amax * 2^e <= 448 (exact float64
    products); 0 for amax == 0, 60 below the fp32 normal range."""
    a = float(np.float32(amax))
    if a == 0.0:
        return 0
    if a < float(np.finfo(np.float32).tiny):
        return 60
    e = 60
    while e > -60 and a * 2.0 ** e > E4M3_MAX:
        e -= 1
    return e


def quantize_do_e4m3_blk(dout: torch.Tensor, seq_offsets, max_seq_len: int):
    """(dO8 uint8 [T, H, D] e4m3 bytes, E8 uint8 [T, H]) for dout [T, H, D]
    (bf16 or fp32).  Tokens past ceil(N/64)*64 of a sequence stay 0."""
    x = dout.detach().float().cpu()
    T, H, D = x.shape
    offs = [int(v) for v in torch.as_tensor(seq_offsets).tolist()]
    y = torch.zeros((T, H, D), dtype=torch.uint8)
    e8 = torch.zeros((T, H), dtype=torch.uint8)
    ntiles = -(-int(max_seq_len) // TILE)
    for b in range(len(offs) - 1):
        st, L = offs[b], offs[b + 1] - offs[b]
        for t in range(ntiles):
            p0 = t * TILE
            if p0 >= L:
                break
            n = min(TILE, L - p0)
            xt = x[st + p0: st + p0 + n]                       # [n, H, D]
            ram = xt.abs().amax(dim=2)                          # [n, H]
            half = torch.as_tensor(group_of(np.arange(n))[1])  # [n]
            for g in (0, 1):
                sel = half == g
                if not bool(sel.any()):
                    continue
                amax = ram[sel].amax(dim=0).numpy().astype(np.float32)  # [H]
                e = group_exp(amax)                                     # [H]
                s = torch.as_tensor((2.0 ** e.astype(np.float64)).astype(np.float32))
                rows = torch.nonzero(sel).flatten() + st + p0
                q = (x[rows] * s[None, :, None]).to(torch.float8_e4m3fn)
                y[rows] = q.view(torch.uint8)
                e8[rows] = torch.as_tensor((127 - e).astype(np.uint8))[None, :].expand(len(rows), H)
    return y, e8


def dequantize_do_e4m3_blk(y: torch.Tensor, e8: torch.Tensor) -> torch.Tensor:
    """bf16 [T, H, D] = y (e4m3 bytes or float8) * 2^(E8 - 127)."""
    yf = (y.view(torch.float8_e4m3fn) if y.dtype == torch.uint8 else y).cpu().double()
    s = torch.pow(2.0, e8.cpu().double() - 127.0)[:, :, None]
    return (yf * s).to(torch.bfloat16)
