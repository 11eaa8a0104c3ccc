"""CPU restatement of the full-FP8 attention backward's numerics.

TEST INFRASTRUCTURE ONLY (imported by ``tests/`` and nowhere in the product).

What the reference's production backward does under DLRM_HSTU_FP8_BWD_FULL
(reference paths relative to ``recommendation_v4/hstu/generative_recommenders/``):

* ``ops/flydsl/hstu_flydsl_mha.py:1330-1394`` -- dO arrives as e4m3 with one
  power-of-two scale per (sequence, head, 32-token group) (the quantizer of
  ``hstu_do_fp8_oracle``); dP = dO8 . V^T stays in that scaled domain and
  the group scales are undone inside the dV / dK / dQ products;
* ``:1351-1370`` -- silu and dS carry the kernel's 1 / N, so their e4m3
  pre-scales are N-relative: P8 = e4m3_sat(silu / N * 2^(c+K_SSC)) and dS8 =
  e4m3_sat(dS * 2^(c+K_DSC)), c = ceil(log2 N), K_SSC = 3, K_DSC = -3 by
  default and -5 in the production gin (``yambda_5b.gin:3764-3799``)
  (``prescales``);
* ``ops/flydsl/hstu_bwd_dkdv.py:356-403`` -- all five products on e4m3
  operands: dV = P8^T dO8, dK = dS8^T q8, dQ = dS8 k8 with the dO group
  scale on the dO side.

This build extends the reference's per-tensor ``qkv_scale`` to per-(token,
head) scales: the query scale is folded into the dK operand and the key
scale into the dQ operand before their casts, times the power-of-two
normaliser 2^-E of the largest scale (``pow2_norm``):
dS8k = e4m3_sat(dS' s_q 2^-Eq 2^(c+K_DSC)), dS8q = e4m3_sat(dS' s_k 2^-Ek 2^(c+K_DSC)).
The bias gradient is read back from dS8q.

Functions and what pins them (``tests/test_bwd_fp8full_oracle.py``):

* ``prescales`` -- closed forms at N = 4096, 1000, 2 and at K_DSC = -5.
* ``pow2_norm`` -- s * norm in [1/2, 1) for the largest s, a power of two.
* ``e4m3_sat`` -- torch's RNE float8_e4m3fn conversion (a library routine)
  after a clamp to +-448.
* ``full_fp8_bwd`` -- with ``quantize=False`` (identity casts) it equals
  ``hstu_oracle.hstu_mha_bwd_closed_form`` (itself pinned against autograd);
  with the casts it stays within the e4m3 error of the unquantized
  backward, and a dropped 2^-e group scale or pre-scale fails both checks.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

from . import hstu_oracle as orc

E4M3_MAX = 448.0


def prescales(N: int, ssc_k: int = 3, dsc_k: int = -3) -> Tuple[float, float]:
    """(P pre-scale 2^(c+ssc_k), dS pre-scale 2^(c+dsc_k)) with
    c = ceil(log2 max(N, 2)) (``hstu_flydsl_mha.py:1351-1370``: K = 3 and -3
    by default; the production gin's DSC_K = -5, ``yambda_5b.gin:3799``)."""
    c = max(1, math.ceil(math.log2(max(int(N), 2))))
    return 2.0 ** (c + ssc_k), 2.0 ** (c + dsc_k)


def pow2_norm(max_scale: float) -> float:
    """2^-e with e the frexp exponent of max_scale (1 for 0)."""
    if max_scale <= 0.0:
        return 1.0
    _, e = math.frexp(float(max_scale))
    return 2.0 ** -e


def e4m3_sat(x: torch.Tensor) -> torch.Tensor:
    """e4m3 value of x after saturation, as float64."""
    return x.clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn).to(torch.float64)


def full_fp8_bwd(
    N: int,
    alpha: float,
    q8: torch.Tensor,
    k8: torch.Tensor,
    v8: torch.Tensor,
    sq: torch.Tensor,
    sk: torch.Tensor,
    sv: torch.Tensor,
    seq_offsets: torch.Tensor,
    dout8: torch.Tensor,
    e8: torch.Tensor,
    attn_bias: Optional[torch.Tensor] = None,
    quantize: bool = True,
    max_scales: Optional[Tuple[float, float]] = None,
    ssc_k: int = 3,
    dsc_k: int = -3,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
    """(dq, dk, dv, dbias) of the causal attention with the full-FP8 casts.

    q8, k8, v8: e4m3 (or any float) [T, H, D] with scales sq, sk, sv [T, H]
    (the dequantized value is q8 * sq); dout8 [T, H, D] with e8 uint8 [T, H]
    (dO = dout8 * 2^(e8 - 127)).  Gradients are with respect to the
    dequantized q, k, v and are float64.  ``quantize=False`` skips every cast
    (the exact backward of the same inputs).  ``max_scales`` = (largest q
    scale, largest k scale) of the whole batch when the rows given are a
    sample of it (the normalisers come from the whole batch).  ``ssc_k`` /
    ``dsc_k``: the pre-scale exponents relative to ceil(log2 N)."""
    T, H, D = q8.shape
    if dout8.dtype == torch.uint8:  # raw e4m3 bytes (the quantizer oracle's output)
        dout8 = dout8.view(torch.float8_e4m3fn)
    ssc, dsc = prescales(N, ssc_k, dsc_k) if quantize else (1.0, 1.0)
    cast = e4m3_sat if quantize else (lambda t: t)
    sq, sk, sv = (s.to(torch.float64).expand(T, H) if s.numel() == 1 else s.to(torch.float64) for s in (sq, sk, sv))
    mq, mk = max_scales if max_scales is not None else (float(sq.abs().max()), float(sk.abs().max()))
    nq = pow2_norm(mq) if quantize else 1.0
    nk = pow2_norm(mk) if quantize else 1.0
    dq = torch.zeros(T, H, D, dtype=torch.float64)
    dk = torch.zeros(T, H, D, dtype=torch.float64)
    dv = torch.zeros(T, H, D, dtype=torch.float64)
    db = None if attn_bias is None else torch.zeros(attn_bias.shape, dtype=torch.float64)
    R = None if attn_bias is None else (attn_bias.shape[1] + 1) // 2
    offs = [int(x) for x in seq_offsets.tolist()]
    for b in range(len(offs) - 1):
        s0, L = offs[b], min(offs[b + 1] - offs[b], N)
        if L <= 0:
            continue
        ar = torch.arange(L)
        mask = (ar.view(L, 1) >= ar.view(1, L)).to(torch.float64)
        idx = None if attn_bias is None else orc.rel_bias_index(ar.view(L, 1), ar.view(1, L), R)
        for h in range(H):
            rows = slice(s0, s0 + L)
            q8h, k8h, v8h = (t[rows, h].to(torch.float64) for t in (q8, k8, v8))
            sqh, skh, svh = sq[rows, h], sk[rows, h], sv[rows, h]
            qr, kr, vr = q8h * sqh[:, None], k8h * skh[:, None], v8h * svh[:, None]
            do8 = dout8[rows, h].to(torch.float64)
            sdo = torch.pow(2.0, e8[rows, h].to(torch.float64) - 127.0)  # 2^-e per query row
            x = alpha * qr @ kr.T
            if attn_bias is not None:
                x = x + attn_bias[h].to(torch.float64)[idx]
            sig = torch.sigmoid(x)
            p8 = cast(x * sig / N * mask * ssc)
            dp = do8 @ vr.T                                    # in dO8's scaled domain
            ds = dp * sig * (1 + x * (1 - sig)) / N * mask     # dS' (still times 2^e)
            ds8k = cast(ds * sqh[:, None] * (nq * dsc))
            ds8q = cast(ds * skh[None, :] * (nk * dsc))
            dv[rows, h] = (p8 * sdo[:, None]).T @ do8 / ssc
            dk[rows, h] = alpha / (nq * dsc) * (ds8k * sdo[:, None]).T @ q8h
            dq[rows, h] = alpha * sdo[:, None] / (nk * dsc) * (ds8q @ k8h)
            if db is not None:
                dsr = ds8q * sdo[:, None] / (skh[None, :] * (nk * dsc))
                db[h].index_add_(0, idx.reshape(-1), (dsr * mask).reshape(-1))
    return dq, dk, dv, db
