"""CPU oracle for one whole HSTU (STU) layer in FP8 -- BASELINE config 5:
LayerNorm -> UVQK projection -> jagged attention -> LayerNorm(attn) * U *
dropout -> output projection + residual -- forward and backward.

TEST INFRASTRUCTURE ONLY (imported by ``tests/`` and nowhere in the product).

Composition of the pinned restatements in ``hstu_oracle`` (attention, e4m3
quantizers) and ``hstu_ln_oracle`` (LayerNorm * U * dropout, masks), in
float64 with torch autograd, following the layer's dataflow
(``modules/stu.py:567-651``; ``ops/hstu_compute.py:86-144, 290-433``;
``ops/triton/triton_hstu_preprocess_and_attention.py:1206-1289``;
``ops/triton/triton_hstu_linear.py:5109-5330``).  Quantization follows the
FP8 contract: forward values are computed from e4m3 operands (LN output at
s_x, per-column e4m3 weights, V/Q/K at s_qkv, the LN * U output at s_out)
while gradients flow as in the reference's default backward: bf16 dgrad /
wgrad GEMMs on the unquantized weights and the recomputed LN(x) / y, and the
attention backward on the e4m3 V/Q/K values (a straight-through estimator at
each quantizer).  With ``grad_scales`` the output and / or UVQK projection's
dgrad runs as the FP8 backward arm does (``ops/triton/bwd_fp8.py:1347-1395,
2313-2520``): the incoming gradient cast to e5m2 at the given scale, the
weight to per-tensor e4m3 (amax / 448), the wgrad and bias gradient exact --
or, for the sites in ``fp8_wgrad``, the wgrad from the e4m3 activation and
the e5m2 gradient (``fp8_wgrad``, ``ops/triton/fp8_wgrad.py:109-160``).
With ``attention="production"`` the attention step is the reference's
production FP8 pair (``DLRM_HSTU_FP8_FWD_PV=1`` and ``DLRM_HSTU_FP8_BWD_FULL=1``,
``dlrm_v4/train/gin/yambda_5b.gin:3293-3319``): the forward is the FP8 P.V
forward of ``hstu_fwd_pv8_oracle.fwd_pv8`` on the e4m3 V/Q/K at the
per-tensor scale s_qkv, and the backward is ``hstu_bwd_fp8full_oracle.full_fp8_bwd``
on the attention output's gradient rounded to bf16 and block-quantized by
``hstu_do_fp8_oracle.quantize_do_e4m3_blk`` (``ops/flydsl/hstu_flydsl_mha.py:1330-1394``),
with the P / dS pre-scale exponents ``ssc_k`` / ``dsc_k``.
Parity pins: those of the composed functions; the composition itself is
checked for shapes, the residual gradient (= dY) and agreement with plain
autograd when the quantizers are identities; the FP8 dgrad against
``hstu_bwd_fp8_oracle.dgrad`` of the same quantized operands; the production
attention step, with its casts off, against the autograd of the dense
attention (``tests/test_layer_oracle.py``).
"""

from __future__ import annotations

from typing import Optional

import numpy as np
import torch
import torch.nn.functional as F

from oracle import hstu_bwd_fp8_oracle as BO
from oracle import hstu_bwd_fp8full_oracle as FO
from oracle import hstu_do_fp8_oracle as DO
from oracle import hstu_fwd_pv8_oracle as PV
from oracle import hstu_ln_oracle as L
from oracle import hstu_oracle as orc


def _ste(full: torch.Tensor, value: torch.Tensor) -> torch.Tensor:
    """``value`` in the forward, d/d``full`` in the backward."""
    return full + (value - full).detach()


def _q_tensor(v: torch.Tensor, scale: Optional[float]) -> torch.Tensor:
    if scale is None:
        return v.detach()
    return L.e4m3_bytes(v.detach(), 1.0 / scale).double() * scale


def _q_weight_cols(w_kn: torch.Tensor) -> torch.Tensor:
    """Per-column e4m3 weight (amax/448 per output column), dequantized."""
    w8, ws = orc.quantize_e4m3_rows(w_kn.detach().t().contiguous().float())
    return orc.dequantize(w8, ws).double().t()


class _Fp8DgradMatmul(torch.autograd.Function):
    """a @ w in the forward; in the backward d(a) = e5m2(g / s_g) s_g .
    (e4m3(w / s_w) s_w)^T with s_w = amax(w) / 448, and d(w) = a^T g -- or,
    with an activation scale s_a, the FP8 weight gradient
    (e4m3(a / s_a) s_a)^T (e5m2(g / s_g) s_g)."""

    @staticmethod
    def forward(ctx, a, w, s_g, s_a):
        ctx.save_for_backward(a, w)
        ctx.s_g, ctx.s_a = s_g, s_a
        return a @ w

    @staticmethod
    def backward(ctx, g):
        a, w = ctx.saved_tensors
        g8 = (g / ctx.s_g).clamp(-57344.0, 57344.0).to(torch.float8_e5m2)
        ws = float(BO.weight_scale(w))
        w8 = (w.detach() / ws).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
        d_a = BO.dgrad(g8, ctx.s_g, w8, ws)
        if ctx.s_a is None:
            d_w = a.t() @ g
        else:
            a8 = (a.detach() / ctx.s_a).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
            d_w = BO.wgrad(a8, g8, ctx.s_a, ctx.s_g).to(g.dtype)
        return d_a, d_w, None, None


class _ProductionAttention(torch.autograd.Function):
    """The production FP8 attention on dequantized q, k, v [T, H, D] whose
    values are e4m3 codes times the per-tensor scale s.  Forward: the FP8
    P.V forward; backward: the full-FP8 backward on e4m3(bf16(dO)) in pow2
    blocks.  ``quantize=False`` turns every cast off (the dO passes
    unquantized at unit group scale): the exact attention and its gradient."""

    @staticmethod
    def forward(ctx, q, k, v, bias, N, alpha, s, offs, pv_scale, ssc_k, dsc_k, quantize):
        codes = [(t.detach() / s) for t in (q, k, v)]
        if quantize:  # exact e4m3 codes (the straight-through sum can be off by an ulp)
            codes = [c.to(torch.float8_e4m3fn).double() for c in codes]
        st = torch.tensor([s], dtype=torch.float64)
        b = None if bias is None else bias.detach()
        out = PV.fwd_pv8(N, alpha, *codes, st, st, st, offs, attn_bias=b, pv_scale=pv_scale, quantize=quantize)
        ctx.save_for_backward(*codes, *([] if b is None else [b]))
        ctx.cfg = (N, alpha, s, offs, ssc_k, dsc_k, quantize, b is not None)
        return out

    @staticmethod
    def backward(ctx, dout):
        N, alpha, s, offs, ssc_k, dsc_k, quantize, has_b = ctx.cfg
        q8, k8, v8 = ctx.saved_tensors[:3]
        b = ctx.saved_tensors[3] if has_b else None
        if quantize:
            y8, e8 = DO.quantize_do_e4m3_blk(dout.to(torch.bfloat16), offs, N)
        else:
            y8, e8 = dout, torch.full(dout.shape[:2], 127, dtype=torch.uint8)
        st = torch.tensor([s], dtype=torch.float64)
        dq, dk, dv, db = FO.full_fp8_bwd(N, alpha, q8, k8, v8, st, st, st, offs, y8, e8, attn_bias=b,
                                         quantize=quantize, ssc_k=ssc_k, dsc_k=dsc_k)
        return dq, dk, dv, db, None, None, None, None, None, None, None, None


def production_attention(q, k, v, s, offs, N, alpha, attn_bias=None, pv_scale=10.04, ssc_k=3, dsc_k=-3,
                         quantize=True):
    """[T, H, D] float64 output of the production FP8 attention (see
    ``_ProductionAttention``), differentiable in q, k, v and the bias."""
    return _ProductionAttention.apply(q, k, v, attn_bias, N, alpha, float(s), offs, pv_scale, ssc_k, dsc_k,
                                      quantize)


def fp8_dgrad_matmul(a: torch.Tensor, w: torch.Tensor, s_g: Optional[float],
                     s_a: Optional[float] = None) -> torch.Tensor:
    return a @ w if s_g is None else _Fp8DgradMatmul.apply(a, w, s_g, s_a)


def hstu_layer_ref(x, params, lengths, max_seq_len, *, num_heads=4, attn_dim=128, hidden_dim=128, eps=1e-6,
                   alpha=None, s_x=None, s_qkv=None, s_out=None, dropout_ratio=0.0, mask=None, attn_bias=None,
                   quantize=True, grad_scales=None, fp8_wgrad=(), attention="dense", pv_scale=10.04, ssc_k=3,
                   dsc_k=-3):
    """Layer output [T, E] (float64, differentiable w.r.t. x and every
    parameter tensor in ``params``).  ``s_*`` = None with ``quantize`` keeps
    that stage in full precision; ``quantize=False`` disables every
    quantizer.  ``grad_scales``: {"output_projection": s, "uvqk_projection":
    s} -- the e5m2 gradient scale of each projection whose dgrad runs in
    FP8; ``fp8_wgrad``: the sites among those whose weight gradient is the FP8
    product of the e4m3 activation (at s_x / s_out) and the e5m2 gradient;
    ``attention``: "dense" (the float64 attention and its exact gradient on
    the quantized V/Q/K) or "production" (the FP8 P.V forward at
    ``pv_scale`` and the full-FP8 backward at ``ssc_k`` / ``dsc_k``; needs
    ``s_qkv``)."""
    gs = grad_scales or {}
    H, Dq, Dv = num_heads, attn_dim, hidden_dim
    nu = H * Dv
    T = x.shape[0]
    alpha = alpha if alpha is not None else 1.0 / Dq ** 0.5
    p = params
    xn = F.layer_norm(x, (x.shape[1],), p["input_norm_weight"], p["input_norm_bias"], eps)
    uvqk_f = fp8_dgrad_matmul(xn, p["uvqk_weight"], gs.get("uvqk_projection"),
                              s_x if "uvqk_projection" in fp8_wgrad else None) + p["uvqk_bias"]
    if quantize and s_x is not None:
        xq = _q_tensor(xn, s_x)
        uvqk_q = xq @ _q_weight_cols(p["uvqk_weight"]) + p["uvqk_bias"].detach()
    else:
        uvqk_q = uvqk_f.detach()
    # with quantize, the stages the kernels hand over in bf16 (u, a bf16 vqk,
    # attn) are rounded to bf16 as well
    bf = (lambda t: t.to(torch.bfloat16).double()) if quantize else (lambda t: t)
    u = _ste(uvqk_f[:, :nu], bf(uvqk_q[:, :nu]))
    vqk_val = uvqk_q[:, nu:]
    vqk_val = _q_tensor(vqk_val, s_qkv) if (quantize and s_qkv is not None) else bf(vqk_val)
    vqk = _ste(uvqk_f[:, nu:], vqk_val)
    v = vqk[:, :nu].reshape(T, H, Dv)
    q = vqk[:, nu:nu + H * Dq].reshape(T, H, Dq)
    k = vqk[:, nu + H * Dq:].reshape(T, H, Dq)
    offs = orc.offsets_from_lengths(lengths)
    if attention == "production":
        if not (quantize and s_qkv is not None):
            raise ValueError("the production attention runs on e4m3 V/Q/K: give s_qkv with quantize=True")
        attn = production_attention(q, k, v, s_qkv, offs, max_seq_len, alpha, attn_bias=attn_bias,
                                    pv_scale=pv_scale, ssc_k=ssc_k, dsc_k=dsc_k).reshape(T, H * Dv)
    elif attention == "dense":
        attn = orc.hstu_mha_dense(max_seq_len, alpha, q, k, v, offs, attn_bias=attn_bias,
                                  dtype=torch.float64).reshape(T, H * Dv)
    else:
        raise ValueError(f"attention {attention!r}: dense | production")
    attn = _ste(attn, bf(attn.detach()))
    y, _, _ = L.ln_mul_dropout_fwd(attn, u, p["output_norm_weight"], p["output_norm_bias"], eps,
                                   dropout_ratio=dropout_ratio, mask=mask, silu_u=True, concat_u=True,
                                   concat_x=True, mul_u_activation_type="silu")
    W = p["output_weight"]
    full = fp8_dgrad_matmul(y, W, gs.get("output_projection"), s_out if "output_projection" in fp8_wgrad else None)
    if quantize and s_out is not None:
        val = _q_tensor(y, s_out) @ _q_weight_cols(W)
    else:
        val = full.detach()
    return x + _ste(full, val)


def make_layer_params(E=512, H=4, Dq=128, Dv=128, seed=0, dtype=torch.bfloat16):
    """Random-init STU parameters (``modules/stu.py:274-328`` shapes)."""
    g = torch.Generator().manual_seed(seed)
    n_uvqk = 2 * H * (Dq + Dv)
    return {
        "input_norm_weight": (1 + 0.1 * torch.randn(E, generator=g)).to(dtype),
        "input_norm_bias": (0.05 * torch.randn(E, generator=g)).to(dtype),
        "uvqk_weight": (torch.randn(E, n_uvqk, generator=g) / E ** 0.5).to(dtype),
        "uvqk_bias": (0.02 * torch.randn(n_uvqk, generator=g)).to(dtype),
        "output_norm_weight": (1 + 0.1 * torch.randn(H * Dv, generator=g)).to(dtype),
        "output_norm_bias": (0.05 * torch.randn(H * Dv, generator=g)).to(dtype),
        "output_weight": (torch.randn(3 * H * Dv, E, generator=g) / (3 * H * Dv) ** 0.5).to(dtype),
    }


def layer_flops(lengths, E=512, H=4, D=128) -> dict:
    """Algorithmic FLOPs of one layer: the UVQK GEMM 2*T*E*(4*H*D) and the
    output projection 2*T*(3*H*D)*E (forward once, backward twice: dgrad and
    wgrad), attention 4*D*H*P forward and 10*D*H*P backward."""
    T = int(np.sum(lengths))
    gemm_fwd = 2 * T * E * (2 * H * 2 * D) + 2 * T * (3 * H * D) * E
    attn_f = orc.attn_flops(lengths, H, D, fwd=True, bwd=False)
    attn_b = orc.attn_flops(lengths, H, D, fwd=False, bwd=True)
    return {"gemm_fwd": gemm_fwd, "gemm_bwd": 2 * gemm_fwd, "attn_fwd": attn_f, "attn_bwd": attn_b,
            "total": 3 * gemm_fwd + attn_f + attn_b}
