"""CPU oracle of the FP8 P.V attention forward (the reference's
``DLRM_HSTU_FP8_FWD_PV=1`` contract).

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports this file:
only ``tests/`` use it, as the checker of ``hstu_attn_fwd_fp8_pv``.

Reference (paths relative to ``recommendation_v4/hstu/generative_recommenders/``):

* ``ops/flydsl/hstu_flydsl_mha.py:2199-2330`` -- the switch and the static P
  scale ``s`` (``DLRM_HSTU_FP8_FWD_PV_SCALE``: unset = 10.04, ``pow2``/``0`` =
  2^3, else a float in [4, 32]);
* ``ops/flydsl/hstu_fwd.py:253-283, 579-589, 1110-1131`` -- the cast: with
  x' = -log2(e) x the exp2-domain SiLU is P' = x' / (1 + 2^x'), the kernel
  stores P8 = e4m3(sat(P' s)) and multiplies the output by 1 / s (and by the
  per-tensor V scale, which rides on the accumulator);
* ``dlrm_v4/train/gin/yambda_5b.gin:3293-3319`` -- the production default.

The reference takes one per-tensor ``qkv_scale``.  For per-(token, head) V
scales this build folds r_k = s_v(k) 2^-E(k) into P before the cast, E(k)
the frexp exponent of the largest V scale among the keys of k's group: the
keys of the same 64-key tile (tiles start at the sequence start) with the same
bit 4 of their index in the tile; the kernel returns 2^E(k) as the E8M0 block
scale of its P.V MFMA.  With one per-tensor scale r_k = 1.

Pinning (``tests/test_fwd_pv8_oracle.py``):

* ``fwd_pv8(quantize=False)`` equals the pinned float64 attention
  (``hstu_oracle.hstu_mha_dense`` on the dequantized inputs) to 1e-12, for
  per-tensor and per-token scales, with and without bias: this pins the
  exp2-domain SiLU, the output scale, the identity r_k 2^E(k) = s_v(k) and the
  causal mask;
* the group exponents against a brute-force loop over (tile, group) on tiny
  inputs, and the closed form 0.5 <= max_group r_k < 1;
* with the cast, the error against the unquantized forward stays within the
  e4m3 bound (3.5e-2 relative L2; 2.6 % measured), and a planted mistake (P
  cast to e5m2) breaks it.
"""

from __future__ import annotations

import math
from typing import Optional

import torch

from oracle import hstu_oracle as orc

LOG2E = 1.4426950408889634
LN2 = 0.6931471805599453


def e4m3_sat(x: torch.Tensor) -> torch.Tensor:
    """Round-to-nearest-even e4m3 of x clamped to +-448, as float64."""
    return x.clamp(-448.0, 448.0).to(torch.float8_e4m3fn).to(torch.float64)


def group_exponents(sv_head: torch.Tensor, L: int) -> torch.Tensor:
    """E(k) for the keys 0..L-1 of one (sequence, head): the frexp exponent of
    the largest V scale over k's group (64-key tile, bit 4 of the index in the
    tile); 0 for an all-zero group."""
    E = torch.zeros(L, dtype=torch.float64)
    for t0 in range(0, L, 64):
        for g in (0, 1):
            idx = [k for k in range(t0, min(t0 + 64, L)) if ((k - t0) >> 4) & 1 == g]
            if not idx:
                continue
            m = float(sv_head[idx].max())
            e = math.frexp(m)[1] if m > 0 else 0
            E[idx] = float(e)
    return E


def fwd_pv8(
    N: int,
    alpha: float,
    q8: torch.Tensor,
    k8: torch.Tensor,
    v8: torch.Tensor,
    sq: torch.Tensor,
    sk: torch.Tensor,
    sv: torch.Tensor,
    seq_offsets: torch.Tensor,
    attn_bias: Optional[torch.Tensor] = None,
    pv_scale: float = 10.04,
    quantize: bool = True,
) -> torch.Tensor:
    """float64 [T, H, D] output of the FP8 P.V forward, causal mask.  q8/k8/v8
    e4m3 [T, H, D]; sq/sk/sv one per-tensor scale (numel 1) or [T, H]."""
    T, H, D = q8.shape
    per_tensor = sv.numel() == 1
    out = torch.zeros(T, H, D, dtype=torch.float64)

    def sc(s, r0, r1, h):
        s = s.double()
        return s.reshape(-1)[0].expand(r1 - r0) if s.numel() == 1 else s[r0:r1, h]

    offs = [int(x) for x in seq_offsets]
    R = 0 if attn_bias is None else (attn_bias.shape[1] + 1) // 2
    for b in range(len(offs) - 1):
        r0, r1 = offs[b], offs[b + 1]
        L = min(r1 - r0, N)
        r1 = r0 + L
        if L == 0:
            continue
        i = torch.arange(L).view(-1, 1)
        j = torch.arange(L).view(1, -1)
        causal = j <= i
        for h in range(H):
            qd = q8[r0:r1, h].double() * sc(sq, r0, r1, h).view(-1, 1)
            kd = k8[r0:r1, h].double() * sc(sk, r0, r1, h).view(-1, 1)
            S = alpha * (qd @ kd.t())
            if attn_bias is not None:
                S = S + attn_bias[h].double()[orc.rel_bias_index(i, j, R)]
            x = -LOG2E * S
            Pp = x / (1.0 + torch.exp2(x))              # P' = -log2(e) silu(S)
            Pp = torch.where(causal, Pp, torch.zeros_like(Pp))
            svh = sc(sv, r0, r1, h)
            if per_tensor:  # r_k = 1, the V scale rides on the output
                r = torch.ones(L, dtype=torch.float64)
                vscale = torch.full((L,), float(svh[0]), dtype=torch.float64)
            else:  # r_k = s_v(k) 2^-E(k), 2^E(k) back on V
                E = group_exponents(svh, L)
                r = svh * torch.exp2(-E)
                vscale = torch.exp2(E)
            P8 = Pp * pv_scale * r.view(1, -1)
            if quantize:
                P8 = e4m3_sat(P8)
            vv = v8[r0:r1, h].double() * vscale.view(-1, 1)
            out[r0:r1, h] = (P8 @ vv) * (-LN2 / (pv_scale * N))
    return out
