"""The HSTU layer's input side -- LayerNorm -> UVQK projection -> jagged
attention -- and the whole layer, on this build's kernels.

Drop-in names (reference file:line, relative to
``recommendation_v4/hstu/generative_recommenders/``):

* ``triton_hstu_preprocess_and_attention`` <- ``ops/triton/triton_hstu_preprocess_and_attention.py:3328-3393``
  (``_HSTUPreprocessAndAttentionFunction``, :1039-2355)
* ``hstu_preprocess_and_attention``        <- ``ops/hstu_compute.py:290-433``
* ``hstu_compute_uqvk``                    <- ``ops/hstu_compute.py:86-144``

FP8 forward (``fp8_input_scale`` given, as :1206-1289 with the fused-LN and
fused-QKV switches on): x8 = e4m3(LN(x) / s_x) from the LayerNorm kernel;
U = bf16(x8 W8_u s_x s_w + b_u) (SiLU fused unless ``defer_silu``); with
``fp8_qkv_scale`` VQK = e4m3((x8 W8_vqk s_x s_w + b) / s_qkv) and the FP8
attention reads V, Q, K in place from that buffer at scale s_qkv, else VQK is
bf16.  Backward: the attention backward writes dV, dQ, dK into one d(uvqk)
[T, 2048] buffer whose U columns the output block's LN * U backward already
filled (``du_row_width``, as :227-260 adopt it), then the dgrad / wgrad
GEMMs on the recomputed bf16 LN(x) -- bf16, or with ``DLRM_HSTU_FP8_BWD_UVQK=1``
the e5m2 dgrad of ``bwd_fp8.uvqk_projection_backward`` (:2180-2300 call it) --
and the LayerNorm backward.
"""

from __future__ import annotations

import logging
from typing import Optional, Tuple

import torch
import torch.nn.functional as F

from . import bwd_fp8
from . import fp8 as _fp8
from .hstu_attention import HammerKernel, hstu_mha, triton_hstu_attention_bwd, triton_hstu_attention_fwd
from .hstu_linear import _ln_bwd, _ln_fwd, hstu_compute_output
from .wgrad import token_wgrad

DUVQK_WIDTH_ATTR = "_hstu_duvqk_width"
logger = logging.getLogger(__name__)


def _adopt_duvqk(du: Optional[torch.Tensor], T: int, width: int, like: torch.Tensor) -> torch.Tensor:
    """The d(uvqk) buffer: ``du`` itself when it is the leading columns of a
    [T, width] row-major buffer (the output block allocated it so), else a
    fresh buffer with du copied in."""
    if (du is not None and du.dim() == 2 and du.shape[0] == T and du.stride() == (width, 1)
            and du.untyped_storage().nbytes() >= (du.storage_offset() + T * width) * du.element_size()):
        return du.as_strided((T, width), (width, 1), du.storage_offset())
    buf = torch.empty((T, width), dtype=like.dtype, device=like.device)
    if du is None:
        buf[:, : like.shape[1]].zero_()
    else:
        buf[:, : du.shape[1]].copy_(du)
    return buf


class _HSTUPreprocessAndAttentionFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, norm_weight, norm_bias, norm_eps, num_heads, attn_dim, hidden_dim, uvqk_weight, uvqk_bias,
                max_seq_len, seq_offsets, attn_alpha, num_targets, max_attn_len, contextual_seq_len,
                fp8_input_scale, fp8_qkv_scale, defer_silu, attn_bias, fp8_backward=None, residual_link=None):
        T, E = x.shape
        H, Dq, Dv = num_heads, attn_dim, hidden_dim
        nu = H * Dv
        # A scale is used once it is ready: a plain scale tensor always, a
        # [2 + steps] state buffer once calibrated; until then this call runs
        # the bf16 path and is one calibration step (triton_hstu_preprocess_and_attention.py:1300-1350).
        # Scales stay on the device: the kernels read them there.
        use_fp8 = _fp8.scale_ready(fp8_input_scale)
        use_fp8_qkv = use_fp8 and _fp8.scale_ready(fp8_qkv_scale)
        calibrate_qkv = fp8_qkv_scale is not None and not use_fp8_qkv
        sa = None
        if use_fp8:
            sa = _fp8.fp8_scale_tensor(fp8_input_scale).reshape(1)
            x8, mean, rstd, _ = _ln_fwd(x, None, norm_weight, norm_bias, norm_eps, 0.0, False, False, False, False,
                                        "none", 0, True, 1.0, out_scale=sa)
            u = _fp8.fp8_gemm(x8, sa, uvqk_weight[:, :nu], bias=uvqk_bias[:nu],
                              silu_cols=None if defer_silu else (0, nu))
            if use_fp8_qkv:
                qkv_scale = _fp8.fp8_scale_tensor(fp8_qkv_scale).reshape(1)
                vqk = _fp8.fp8_gemm(x8, sa, uvqk_weight[:, nu:], bias=uvqk_bias[nu:], out_dtype=_fp8.E4M3,
                                    out_scale=qkv_scale)
            else:
                vqk = _fp8.fp8_gemm(x8, sa, uvqk_weight[:, nu:], bias=uvqk_bias[nu:])
                qkv_scale = None
            u_pre = None
        else:
            xn, mean, rstd, _ = _ln_fwd(x, None, norm_weight, norm_bias, norm_eps, 0.0, False, False, False, False,
                                        "none", 0, False, 1.0)
            if fp8_input_scale is not None:
                _fp8.calibrate_scale_buffer(fp8_input_scale, xn)
            uvqk = _fp8.proj_mm(xn, uvqk_weight.to(x.dtype).t(), bias=uvqk_bias)
            u_pre = uvqk[:, :nu]
            u = u_pre if defer_silu else F.silu(u_pre)
            vqk = uvqk[:, nu:]
            qkv_scale = None
        if calibrate_qkv:
            _fp8.calibrate_scale_buffer(fp8_qkv_scale, vqk)
        v = vqk[:, :nu].view(T, H, Dv)
        q = vqk[:, nu:nu + H * Dq].view(T, H, Dq)
        k = vqk[:, nu + H * Dq:].view(T, H, Dq)
        attn = triton_hstu_attention_fwd(max_seq_len, attn_alpha, q, k, v, seq_offsets, num_targets, max_attn_len,
                                         contextual_seq_len, None, False, 0, qkv_scale, qkv_scale, qkv_scale,
                                         attn_bias=attn_bias)
        # the e4m3 LN output feeds the FP8 UVQK weight gradient (fp8t switch)
        keep_x8 = use_fp8 and bwd_fp8.uvqk_wgrad_fp8t(fp8_backward)
        ctx.save_for_backward(x, norm_weight, norm_bias, mean, rstd, uvqk_weight, vqk, seq_offsets,
                              *([] if num_targets is None else [num_targets]),
                              *([] if attn_bias is None else [attn_bias]),
                              *([] if u_pre is None else [u_pre]),
                              *([x8] if keep_x8 else []))
        ctx.cfg = (norm_eps, H, Dq, Dv, max_seq_len, attn_alpha, max_attn_len, contextual_seq_len, qkv_scale,
                   defer_silu, num_targets is not None, attn_bias is not None, u_pre is not None)
        ctx.x8_scale = sa if keep_x8 else None
        ctx.fp8_backward = fp8_backward
        ctx.residual_link = residual_link
        if residual_link is not None:
            residual_link.bind(x)
        u = u.contiguous() if u.stride(1) != 1 else u
        setattr(u, DUVQK_WIDTH_ATTR, uvqk_weight.shape[1])
        return u, attn.view(T, H * Dv)

    @staticmethod
    def backward(ctx, du, dattn):
        (eps, H, Dq, Dv, N, alpha, max_attn_len, ctx_len, qkv_scale, defer_silu, has_nt, has_bias,
         has_upre) = ctx.cfg
        saved = list(ctx.saved_tensors)
        x, nw, nb, mean, rstd, W, vqk, seq_offsets = saved[:8]
        i = 8
        num_targets = saved[i] if has_nt else None
        i += int(has_nt)
        attn_bias = saved[i] if has_bias else None
        i += int(has_bias)
        u_pre = saved[i] if has_upre else None
        i += int(has_upre)
        x8 = saved[i] if ctx.x8_scale is not None else None
        T = x.shape[0]
        nu = H * Dv
        width = W.shape[1]
        duvqk = _adopt_duvqk(du, T, width, x)
        if not defer_silu:
            if u_pre is None:
                raise NotImplementedError("SiLU-fused FP8 U needs defer_silu=True for its backward")
            sg = torch.sigmoid(u_pre.float())
            duvqk[:, :nu] = (duvqk[:, :nu].float() * sg * (1 + u_pre.float() * (1 - sg))).to(x.dtype)
        v = vqk[:, :nu].view(T, H, Dv)
        q = vqk[:, nu:nu + H * Dq].view(T, H, Dq)
        k = vqk[:, nu + H * Dq:].view(T, H, Dq)
        dv = duvqk[:, nu:2 * nu].view(T, H, Dv)
        dq = duvqk[:, 2 * nu:2 * nu + H * Dq].view(T, H, Dq)
        dk = duvqk[:, 2 * nu + H * Dq:].view(T, H, Dq)
        dbias = None
        if attn_bias is not None:
            dbias = torch.empty(attn_bias.shape, dtype=torch.float32, device=x.device)
        bcfg = bwd_fp8.resolve(ctx.fp8_backward)
        triton_hstu_attention_bwd(dattn.contiguous().view(T, H, Dv), q, k, v, dq, dk, dv, seq_offsets, num_targets,
                                  N, alpha, max_attn_len, ctx_len, None, False, 0, qkv_scale, qkv_scale, qkv_scale,
                                  attn_bias=attn_bias, dbias=dbias,
                                  full_fp8=bcfg.attn_full_fp8, ssc_k=bcfg.attn_ssc_k, dsc_k=bcfg.attn_dsc_k)
        # projection backward on the recomputed bf16 LN(x): the FP8 dgrad arm
        # (DLRM_HSTU_FP8_BWD_UVQK=1, after its warm-up), else bf16 GEMMs
        def recompute_normed_x() -> torch.Tensor:
            return _ln_fwd(x, None, nw, nb, eps, 0.0, False, False, False, False, "none", 0, False, 1.0)[0]

        fp8_grads = bwd_fp8.uvqk_projection_backward(duvqk, None, ctx.x8_scale, W, normed_x_fp8_t=x8,
                                                     recompute_normed_x=recompute_normed_x,
                                                     config=ctx.fp8_backward)
        if fp8_grads is not None:
            dxn, d_w, d_b = fp8_grads
        else:
            xn = recompute_normed_x()
            # the wgrad kernel also sums d(uvqk)'s columns: the bias gradient
            d_w, d_b = token_wgrad(xn, duvqk, with_colsum=True)
            dxn = _fp8.proj_mm(duvqk, W)
        d_w, d_b = d_w.to(W.dtype), d_b.to(W.dtype)
        # the output block's residual gradient of x, when the layer linked it,
        # is added inside the LayerNorm backward
        dres = None if ctx.residual_link is None else ctx.residual_link.take()
        dx, _, dnw, dnb, _ = _ln_bwd(dxn, x, None, nw, nb, mean, rstd, 0.0, None, False, False, False, "none", False,
                                     dres=dres)
        return (dx, dnw.to(nw.dtype), dnb.to(nb.dtype), None, None, None, None, d_w, d_b, None, None, None, None,
                None, None, None, None, None, None if dbias is None else dbias.to(attn_bias.dtype), None, None)


def triton_hstu_preprocess_and_attention(
    x: torch.Tensor,
    norm_weight: torch.Tensor,
    norm_bias: torch.Tensor,
    norm_eps: float,
    num_heads: int,
    attn_dim: int,
    hidden_dim: int,
    uvqk_weight: torch.Tensor,
    uvqk_bias: torch.Tensor,
    max_seq_len: int,
    seq_offsets: torch.Tensor,
    attn_alpha: float,
    num_targets: Optional[torch.Tensor],
    max_attn_len: int = 0,
    contextual_seq_len: int = 0,
    recompute_uvqk_in_backward: bool = False,
    recompute_normed_x_in_backward: bool = False,
    sort_by_length: bool = False,
    enable_tma: Optional[bool] = None,
    fp8_input_scale: Optional[torch.Tensor] = None,
    fp8_qkv_scale: Optional[torch.Tensor] = None,
    defer_silu: bool = False,
    allow_save_fp8_uvqk: bool = True,
    return_residual_proxy: bool = False,
    *,
    attn_bias: Optional[torch.Tensor] = None,
    fp8_backward: Optional[bwd_fp8.Fp8BackwardConfig] = None,
    residual_link=None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """(u, attn [T, H*hidden_dim]); signature of
    ``triton_hstu_preprocess_and_attention`` (:3328-3393).  ``attn_bias`` is
    this build's relative-position bias extension (default off);
    ``fp8_backward`` the FP8 backward arm's settings (default: the process
    default, ``bwd_fp8.default_config()``); ``residual_link``
    (``hstu_linear.ResidualLink``): the same layer's output block hands its
    residual gradient of x over it.  ``fp8_input_scale`` /
    ``fp8_qkv_scale``: one-element device scales, or the reference's
    [2 + steps] scale state buffers, calibrated by the bf16 calls until frozen."""
    if return_residual_proxy:
        raise NotImplementedError("the residual-proxy dropout fold is not served")
    if fp8_input_scale is None and fp8_qkv_scale is not None:
        raise ValueError("fp8_qkv_scale needs fp8_input_scale (the QKV GEMM reads the e4m3 LN output)")
    return _HSTUPreprocessAndAttentionFunction.apply(
        x, norm_weight, norm_bias, norm_eps, num_heads, attn_dim, hidden_dim, uvqk_weight, uvqk_bias, max_seq_len,
        seq_offsets, attn_alpha, num_targets, max_attn_len, contextual_seq_len, fp8_input_scale, fp8_qkv_scale,
        defer_silu, attn_bias, fp8_backward, residual_link)


class _NormProjFunction(torch.autograd.Function):
    """``LN(x) . W + b`` on this build's kernels: the LayerNorm kernel and the
    bf16 GEMM (``ops/hstu_compute.py:108-127`` with a Triton/HIP ``kernel``).
    Backward: the token-axis weight gradient with the bias column sum in the
    same pass, the bf16 dgrad ``d(uvqk) . W^T`` and the LayerNorm backward
    on the saved mean / rstd."""

    @staticmethod
    def forward(ctx, x, norm_weight, norm_bias, norm_eps, uvqk_weight, uvqk_bias):
        xn, mean, rstd, _ = _ln_fwd(x, None, norm_weight, norm_bias, norm_eps, 0.0, False, False, False, False,
                                    "none", 0, False, 1.0)
        w = uvqk_weight.to(x.dtype)
        uvqk = _fp8.bf16_gemm(xn, w.t(), bias=uvqk_bias)
        ctx.save_for_backward(x, norm_weight, norm_bias, mean, rstd, w, xn)
        ctx.dtypes = (uvqk_weight.dtype, uvqk_bias.dtype)
        return uvqk

    @staticmethod
    def backward(ctx, duvqk):
        x, nw, nb, mean, rstd, w, xn = ctx.saved_tensors
        w_dtype, b_dtype = ctx.dtypes
        duvqk = duvqk.to(x.dtype).contiguous()
        d_w, d_b = token_wgrad(xn, duvqk, with_colsum=True)
        dxn = _fp8.bf16_gemm(duvqk, w)
        dx, _, dnw, dnb, _ = _ln_bwd(dxn, x, None, nw, nb, mean, rstd, 0.0, None, False, False, False, "none", False)
        return dx, dnw.to(nw.dtype), dnb.to(nb.dtype), None, d_w.to(w_dtype), d_b.to(b_dtype)


def uqvk_kernel_reason(x: torch.Tensor, norm_weight, norm_bias, uvqk_weight: torch.Tensor,
                       uvqk_bias) -> Optional[str]:
    """Why ``hstu_compute_uqvk`` cannot run on the LayerNorm kernel and the
    bf16 GEMM (None: it can): bf16 device rows, LayerNorm width in
    ``SERVED_D``, projection width a multiple of 256 (the weight gradient's
    tile), both LayerNorm parameters and the bias given."""
    from .hstu_linear import SERVED_D

    if not x.is_cuda or x.dtype != torch.bfloat16 or x.dim() != 2:
        return f"x must be a 2-D bf16 device tensor (got {x.dtype}, {tuple(x.shape)})"
    if x.shape[1] not in SERVED_D:
        return f"LayerNorm width {x.shape[1]} not served (D in {SERVED_D})"
    if norm_weight is None or norm_bias is None or uvqk_bias is None:
        return "the kernel path takes the LayerNorm weight and bias and the projection bias"
    if uvqk_weight.dim() != 2 or uvqk_weight.shape[0] != x.shape[1] or uvqk_weight.shape[1] % 256 != 0:
        return f"uvqk_weight {tuple(uvqk_weight.shape)} not served (K = {x.shape[1]}, N % 256 == 0)"
    return None


_UQVK_LOGGED: set = set()


def hstu_compute_uqvk(x, norm_weight, norm_bias, norm_eps, num_heads, attn_dim, hidden_dim, uvqk_weight, uvqk_bias,
                      kernel: HammerKernel = HammerKernel.PYTORCH):
    """LN -> addmm -> split u|v|q|k -> silu(u) (``ops/hstu_compute.py:86-144``).
    ``kernel=PYTORCH``: torch ops (``F.layer_norm`` + ``torch.addmm``), as the
    reference's PyTorch path.  ``TRITON`` / ``HIP``: this build's LayerNorm
    kernel and bf16 GEMM (``_NormProjFunction``); a shape those kernels do
    not serve takes the torch ops, with the reason logged once.  Returns
    (u, q, k, v), q/k/v as [T, H, D] views of the projection."""
    uvqk = None
    if kernel in (HammerKernel.TRITON, HammerKernel.HIP):
        why = uqvk_kernel_reason(x, norm_weight, norm_bias, uvqk_weight, uvqk_bias)
        if why is None:
            uvqk = _NormProjFunction.apply(x, norm_weight, norm_bias, norm_eps, uvqk_weight, uvqk_bias)
        elif why not in _UQVK_LOGGED:
            _UQVK_LOGGED.add(why)
            logger.warning("hstu_compute_uqvk: %s; the torch ops run", why)
    if uvqk is None:
        xn = F.layer_norm(x, (x.shape[-1],), norm_weight, norm_bias, norm_eps)
        uvqk = torch.addmm(uvqk_bias, xn, uvqk_weight)
    u, v, q, k = torch.split(uvqk, [hidden_dim * num_heads, hidden_dim * num_heads, attn_dim * num_heads,
                                    attn_dim * num_heads], dim=1)
    return (F.silu(u), q.reshape(-1, num_heads, attn_dim), k.reshape(-1, num_heads, attn_dim),
            v.reshape(-1, num_heads, hidden_dim))


def hstu_preprocess_and_attention(
    x, norm_weight, norm_bias, norm_eps, num_heads, attn_dim, hidden_dim, uvqk_weight, uvqk_bias, max_seq_len,
    seq_offsets, attn_alpha, causal, num_targets, max_attn_len, contextual_seq_len, recompute_uvqk_in_backward,
    recompute_normed_x_in_backward, sort_by_length, prefill=False, kernel: HammerKernel = HammerKernel.PYTORCH,
    enable_tma=None, fp8_input_scale=None, fp8_qkv_scale=None, defer_silu=False, allow_save_fp8_uvqk=True,
    return_residual_proxy=False,
):
    """Layer-level dispatch (``ops/hstu_compute.py:290-433``): returns
    (u, attn, k, v) with k = v = None on the fused path."""
    if not causal:
        raise ValueError("only causal attention is supported.")
    if kernel in (HammerKernel.TRITON, HammerKernel.HIP) and not prefill:
        u, attn = triton_hstu_preprocess_and_attention(
            x, norm_weight, norm_bias, norm_eps, num_heads, attn_dim, hidden_dim, uvqk_weight, uvqk_bias,
            max_seq_len, seq_offsets, attn_alpha, num_targets, max_attn_len, contextual_seq_len,
            recompute_uvqk_in_backward, recompute_normed_x_in_backward, sort_by_length, enable_tma,
            fp8_input_scale, fp8_qkv_scale, defer_silu, allow_save_fp8_uvqk, return_residual_proxy)
        return u, attn, None, None
    u, q, k, v = hstu_compute_uqvk(x, norm_weight, norm_bias, norm_eps, num_heads, attn_dim, hidden_dim,
                                   uvqk_weight, uvqk_bias, kernel)
    attn = hstu_mha(max_seq_len, attn_alpha, q, k, v, seq_offsets, True, 0.0, False, num_targets,
                    max_attn_len=max_attn_len, contextual_seq_len=contextual_seq_len, sort_by_length=sort_by_length,
                    kernel=kernel).view(-1, hidden_dim * num_heads)
    return u, attn, k, v


def hstu_layer(
    x: torch.Tensor,
    seq_offsets: torch.Tensor,
    max_seq_len: int,
    params: dict,
    *,
    num_heads: int = 4,
    attn_dim: int = 128,
    hidden_dim: int = 128,
    attn_alpha: Optional[float] = None,
    dropout_ratio: float = 0.0,
    training: bool = True,
    fp8_input_scale: Optional[torch.Tensor] = None,
    fp8_qkv_scale: Optional[torch.Tensor] = None,
    fp8_output_scale: Optional[torch.Tensor] = None,
    attn_bias: Optional[torch.Tensor] = None,
    norm_eps: float = 1e-6,
    seed: Optional[int] = None,
    fp8_backward: Optional[bwd_fp8.Fp8BackwardConfig] = None,
    dropout_mask16: Optional[bool] = None,
) -> torch.Tensor:
    """One STU layer as ``modules/stu.py:567-651`` composes it with the
    production flags (defer_silu; output block with concat_u, concat_x and
    SiLU on u): preprocess + attention, then LN(attn) * U * dropout -> output
    projection + residual.  ``params``: input_norm_weight/bias [E],
    uvqk_weight [E, 2048], uvqk_bias [2048], output_norm_weight/bias
    [H*hidden], output_weight [3*H*hidden, E].

    FP8 scales (``fp8_input_scale``, ``fp8_qkv_scale``, ``fp8_output_scale``)
    are one-element device tensors or the reference's per-layer scale state
    buffers ([2 + steps] fp32, ``fp8.fp8_scale_state_size()``), which the
    first calls calibrate (bf16 math) until frozen; no scale is read on the
    host.  ``fp8_backward`` sets the FP8 backward arm (default: the process
    default); ``dropout_mask16`` the dropout mask scheme (default: the
    process default, ``hstu_linear.set_mask16``)."""
    from .hstu_linear import ResidualLink, triton_hstu_compute_output

    # x's residual gradient joins its LayerNorm backward's dx in one kernel
    link = ResidualLink()
    alpha = attn_alpha if attn_alpha is not None else 1.0 / attn_dim ** 0.5
    u, attn = triton_hstu_preprocess_and_attention(
        x, params["input_norm_weight"], params["input_norm_bias"], norm_eps, num_heads, attn_dim, hidden_dim,
        params["uvqk_weight"], params["uvqk_bias"], max_seq_len, seq_offsets, alpha, None,
        recompute_uvqk_in_backward=True, recompute_normed_x_in_backward=True,
        fp8_input_scale=fp8_input_scale, fp8_qkv_scale=fp8_qkv_scale, defer_silu=True, attn_bias=attn_bias,
        fp8_backward=fp8_backward, residual_link=link)
    return triton_hstu_compute_output(
        attn, u, x, params["output_norm_weight"], params["output_norm_bias"], params["output_weight"], norm_eps,
        dropout_ratio, training, True, True, True, "silu", seed=seed, recompute_y_in_backward=True,
        fp8_output_scale=fp8_output_scale, fp8_backward=fp8_backward, dropout_mask16=dropout_mask16,
        residual_link=link)


__all__ = ["triton_hstu_preprocess_and_attention", "hstu_preprocess_and_attention", "hstu_compute_uqvk",
           "hstu_layer", "hstu_compute_output"]
