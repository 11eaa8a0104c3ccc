"""The HSTU output block -- LayerNorm * U * dropout, the [u | x | y] concat and
the output projection with its residual -- and the weighted LayerNorm, on this
build's gfx950 kernels (``hstu_ln_mul_fwd`` / ``hstu_ln_mul_bwd`` /
``hstu_dropout_mask`` in ``libhstu_mi355x.so``).

Drop-in names (reference file:line, relative to
``recommendation_v4/hstu/generative_recommenders/``):

* ``triton_layer_norm_mul_dropout_fwd`` <- ``ops/triton/triton_hstu_linear.py:3034-3146``
* ``triton_layer_norm_mul_dropout_bwd`` <- ``triton_hstu_linear.py:3689-3747``
* ``triton_norm_mul_dropout``           <- ``triton_hstu_linear.py:6446-6491``
  (``LayerNormMulDropoutFunction``, :3953-4058)
* ``triton_hstu_compute_output``        <- ``triton_hstu_linear.py:6494-6572``
  (``HSTUComputeOutputFunction``, :5109-5900)
* ``hstu_compute_output``               <- ``ops/hstu_compute.py:147-215``
* ``triton_weighted_layer_norm_fwd`` / ``_bwd`` <- ``ops/triton/triton_layer_norm.py:1668-1740, 3574-3640``

Dropout follows the reference's separated-mask path (the one it runs on
gfx950): an int8 mask [N, D] with one keep bit per concatenated block (bit 0 =
y, then x, then u), drawn from Philox4x32-10 with the reference's counters,
in the 32-bit scheme or, with ``set_mask16(True)`` (the process default
comes from ``DLRM_HSTU_FP8_MASK16=1``, as ``yambda_5b.gin`` sets it), the
16-bit-half scheme -- the same bits for the same seed.  The mask is returned by the forward and reused by the backward.

Not served (raise ``NotImplementedError``): group norm, ``rng_row_indices``
(compact last-layer rows), precomputed mean/rstd, the weighted LayerNorm
backward's residual / dropout-mask folds, D other than 256 or 512.
"""

from __future__ import annotations

import os
import weakref
from typing import Optional, Tuple

import torch

from . import _lib, bwd_fp8
from . import fp8 as _fp8
from .wgrad import fp8_wgrad, token_wgrad
from .hstu_attention import HammerKernel
from .pt_hstu_linear import pytorch_hstu_compute_output, pytorch_norm_mul_dropout

E4M3 = torch.float8_e4m3fn
_ACT = {"none": 0, "silu": 1, "sigmoid": 2}
SERVED_D = (256, 512)


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


_mask16: Optional[bool] = None


def _use_mask16() -> bool:
    """16-bit-half keep decisions (``_use_mask16``, triton_hstu_linear.py:2358-2374):
    the process default, read once from ``DLRM_HSTU_FP8_MASK16``."""
    global _mask16
    if _mask16 is None:
        _mask16 = os.environ.get("DLRM_HSTU_FP8_MASK16", "0") == "1"
    return _mask16


def set_mask16(flag: Optional[bool]) -> None:
    """Set the dropout mask scheme (True: 16-bit halves; None: read the
    environment again on next use)."""
    global _mask16
    _mask16 = flag


def _block_d(D: int) -> int:
    return 1 << max(0, (int(D) - 1).bit_length())


def _num_warps(block_d: int) -> int:
    return min(max(block_d // 256, 1), 8)


def _rows(t: torch.Tensor) -> torch.Tensor:
    """A 2-D view with unit column stride (column slices stay in place)."""
    if t.dim() != 2:
        raise ValueError(f"expected a 2-D tensor, got {tuple(t.shape)}")
    return t if t.stride(1) == 1 else t.contiguous()


def _check_bf16(name: str, t: torch.Tensor) -> None:
    if t.dtype != torch.bfloat16:
        raise NotImplementedError(f"{name}: bf16 only (got {t.dtype})")


def _check_d(D: int) -> None:
    if D not in SERVED_D:
        raise NotImplementedError(f"feature dim {D} not served (D in {SERVED_D})")


def _params(weight: Optional[torch.Tensor], bias: Optional[torch.Tensor], D: int, device):
    """(weight, bias, param dtype code) for the LayerNorm kernels: bf16 or fp32
    parameters go as they are (no conversion kernel per call); anything else,
    or a mix of the two, as fp32 copies."""
    w = torch.ones((D,), dtype=torch.float32, device=device) if weight is None else weight.detach()
    b = torch.zeros((D,), dtype=torch.float32, device=device) if bias is None else bias.detach()
    if w.dtype == b.dtype and w.dtype in (torch.bfloat16, torch.float32):
        w, b = w.contiguous(), b.contiguous()
    else:
        w, b = w.to(torch.float32).contiguous(), b.to(torch.float32).contiguous()
    # the kernels read them as 16-byte vectors
    w = w if w.data_ptr() % 16 == 0 else w.clone()
    b = b if b.data_ptr() % 16 == 0 else b.clone()
    return w, b, _lib.HSTU_DTYPE_BF16 if w.dtype == torch.bfloat16 else _lib.HSTU_DTYPE_FP32


def _seed(seed: Optional[int], training: bool) -> int:
    if seed is None and training:
        seed = int(torch.randint(low=0, high=2 ** 62, size=(1,), dtype=torch.int64).item())
    return 0 if seed is None else int(seed)


def _ncols(concat_u: bool, concat_x: bool) -> int:
    return 1 + int(concat_u) + int(concat_x)


def create_dropout_mask(N: int, D: int, concat_u: bool, concat_x: bool, dropout_ratio: float, seed: int,
                        device, mask16: Optional[bool] = None) -> torch.Tensor:
    """int8 [N, D] keep mask, bit j = mask j (``_create_dropout_mask``,
    triton_hstu_linear.py:2547-2600); ``mask16`` None = the process default."""
    mask16 = _use_mask16() if mask16 is None else bool(mask16)
    _check_d(D)
    mask = torch.empty((N, D), dtype=torch.int8, device=device)
    if N == 0:
        return mask
    st = _lib.fn("hstu_dropout_mask")(N, D, _ncols(concat_u, concat_x), int(mask16), float(dropout_ratio),
                                      int(seed) & 0xFFFFFFFFFFFFFFFF, mask.data_ptr(), D,
                                      torch.cuda.current_stream(device).cuda_stream)
    _lib.check(st, "hstu_dropout_mask")
    return mask


# ---------------------------------------------------------------------------
# LayerNorm * U * dropout
# ---------------------------------------------------------------------------
def _ln_fwd(x, u, weight, bias, eps, dropout_ratio, training, silu_u, concat_u, concat_x, act, seed,
            output_fp8, inv_scale, out_scale: Optional[torch.Tensor] = None, mask16: Optional[bool] = None):
    """The LN * U * dropout kernel.  An e4m3 output is scaled by ``inv_scale``
    (host float) or, with ``out_scale`` (a device fp32 scale tensor), by
    1 / out_scale[0] read on the device.  ``mask16`` None = the process default."""
    mask16 = _use_mask16() if mask16 is None else bool(mask16)
    x = _rows(x)
    _check_bf16("x", x)
    N, D = x.shape
    _check_d(D)
    if u is not None:
        u = _rows(u)
        _check_bf16("u", u)
        if u.shape != x.shape:
            raise ValueError(f"u {tuple(u.shape)} must match x {tuple(x.shape)}")
    if act not in _ACT:
        raise ValueError(f"mul_u_activation_type {act!r}")
    cu = bool(concat_u) and u is not None
    ncols = _ncols(cu, concat_x)
    y = torch.empty((N, ncols * D), dtype=E4M3 if output_fp8 else x.dtype, device=x.device)
    mean = torch.empty((N,), dtype=torch.float32, device=x.device)
    rstd = torch.empty((N,), dtype=torch.float32, device=x.device)
    dropout = bool(training) and dropout_ratio > 0.0
    mask = torch.empty((N, D), dtype=torch.int8, device=x.device) if dropout else None
    if N == 0:
        return y, mean, rstd, mask
    w, b, pd = _params(weight, bias, D, x.device)
    st = _lib.fn("hstu_ln_mul_fwd")(
        x.data_ptr(), x.stride(0), _lib.ptr(u), 0 if u is None else u.stride(0), w.data_ptr(), b.data_ptr(), pd,
        float(eps), N, D, _ACT[act], int(bool(silu_u)), int(cu), int(bool(concat_x)), int(dropout),
        float(dropout_ratio), int(seed) & 0xFFFFFFFFFFFFFFFF, int(mask16), _lib.ptr(mask), D,
        y.data_ptr(), y.stride(0), _lib.HSTU_DTYPE_FP8_E4M3 if output_fp8 else _lib.HSTU_DTYPE_BF16,
        float(inv_scale), _lib.ptr(out_scale), mean.data_ptr(), rstd.data_ptr(), _stream(x))
    _lib.check(st, "hstu_ln_mul_fwd")
    return y, mean, rstd, mask


def triton_layer_norm_mul_dropout_fwd(
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
    seed: Optional[int] = None,
    rng_row_indices: Optional[torch.Tensor] = None,
    output_fp8: bool = False,
    inv_scale: float = 1.0,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, int, int, int, Optional[torch.Tensor]]:
    """(y, mean, rstd, BLOCK_D, num_warps, seed, random_mask); random_mask is
    the int8 keep mask when dropout ran, else None."""
    if rng_row_indices is not None:
        raise NotImplementedError("rng_row_indices (compact rows) is not served")
    seed = _seed(seed, training)
    y, mean, rstd, mask = _ln_fwd(x, u, weight, bias, eps, dropout_ratio, training, silu_u, concat_u, concat_x,
                                  mul_u_activation_type, seed, output_fp8, inv_scale)
    bd = _block_d(x.shape[1])
    return y, mean, rstd, bd, _num_warps(bd), seed, mask


def _alloc_du(u: torch.Tensor, du_row_width: int) -> torch.Tensor:
    """du, optionally as the leading columns of a wider row
    (``_alloc_du``, triton_hstu_linear.py:3448-3465)."""
    if du_row_width > u.shape[1] and u.shape[0] > 0:
        return torch.empty((u.shape[0], du_row_width), dtype=u.dtype, device=u.device)[:, : u.shape[1]]
    return torch.empty(u.shape, dtype=u.dtype, device=u.device)


def _ln_bwd(dy, x, u, weight, bias, mean, rstd, dropout_ratio, mask, silu_u, concat_u, concat_x, act,
            compute_y, du_row_width=0, dres=None):
    """The LN * U * dropout backward.  ``dres``: a residual branch's bf16
    gradient of x, added to dx inside the kernel (no x block, no mask)."""
    x = _rows(x)
    dy = _rows(dy)
    _check_bf16("dy", dy)
    N, D = x.shape
    _check_d(D)
    if u is not None:
        u = _rows(u)
    cu = bool(concat_u) and u is not None
    ncols = _ncols(cu, concat_x)
    if dy.shape != (N, ncols * D):
        raise ValueError(f"dy {tuple(dy.shape)}; expected {(N, ncols * D)}")
    dx = torch.empty((N, D), dtype=x.dtype, device=x.device)
    du = None if u is None else _alloc_du(u, du_row_width)
    y = torch.empty((N, ncols * D), dtype=x.dtype, device=x.device) if compute_y else None
    dw = torch.empty((D,), dtype=torch.float32, device=x.device)
    db = torch.empty((D,), dtype=torch.float32, device=x.device)
    w, b, pd = _params(weight, bias, D, x.device)
    if mask is not None:
        mask = _rows(mask)
    if dres is not None:
        dres = _rows(dres)
        _check_bf16("dres", dres)
        if dres.shape != (N, D):
            raise ValueError(f"dres {tuple(dres.shape)}; expected {(N, D)}")
    nbytes = int(_lib.fn("hstu_ln_mul_bwd_workspace_bytes")(N, D))
    ws = torch.empty((nbytes,), dtype=torch.uint8, device=x.device)
    st = _lib.fn("hstu_ln_mul_bwd")(
        dy.data_ptr(), dy.stride(0), x.data_ptr(), x.stride(0), _lib.ptr(u), 0 if u is None else u.stride(0),
        w.data_ptr(), b.data_ptr(), pd, mean.contiguous().data_ptr(), rstd.contiguous().data_ptr(), N, D, _ACT[act],
        int(bool(silu_u)), int(cu), int(bool(concat_x)), float(dropout_ratio), _lib.ptr(mask),
        0 if mask is None else mask.stride(0), dx.data_ptr(), dx.stride(0), _lib.ptr(du),
        0 if du is None else du.stride(0), _lib.ptr(y), 0 if y is None else y.stride(0), _lib.ptr(dres),
        0 if dres is None else dres.stride(0), dw.data_ptr(), db.data_ptr(), ws.data_ptr(), nbytes, _stream(x))
    _lib.check(st, "hstu_ln_mul_bwd")
    return dx, du, dw, db, y


def _outproj_ln_bwd(g8, g_scale, w8, w_scale, x, u, weight, bias, mean, rstd, dropout_ratio, mask, silu_u, act,
                    du_row_width=0):
    """The output projection's FP8 dgrad fused with the LN * U * dropout
    backward ([u' | x | y] concat, D = 512): dy = g8 . w8^T * (s_g s_w) never
    leaves the kernel.  Returns (dx, du, dweight fp32, dbias fp32); dx and du
    equal the unfused dgrad + ``_ln_bwd`` bit for bit."""
    x = _rows(x)
    u = _rows(u)
    N, D = x.shape
    if D != 512 or tuple(w8.shape) != (3 * D, 512) or tuple(g8.shape) != (N, 512):
        raise ValueError(f"fused output-projection backward: x {tuple(x.shape)}, g8 {tuple(g8.shape)}, "
                         f"w8 {tuple(w8.shape)}")
    dx = torch.empty((N, D), dtype=x.dtype, device=x.device)
    du = _alloc_du(u, du_row_width)
    dw = torch.empty((D,), dtype=torch.float32, device=x.device)
    db = torch.empty((D,), dtype=torch.float32, device=x.device)
    w, b, pd = _params(weight, bias, D, x.device)
    if mask is not None:
        mask = _rows(mask)
    g8 = _rows(g8)  # column slices stay in place (row stride = ldg)
    w8 = w8.contiguous()
    gs = g_scale.to(torch.float32).reshape(-1)[:1].contiguous()
    ws_ = w_scale.to(torch.float32).reshape(-1)[:1].contiguous()
    nbytes = int(_lib.fn("hstu_outproj_ln_bwd_workspace_bytes")(N))
    ws = torch.empty((nbytes,), dtype=torch.uint8, device=x.device)
    st = _lib.fn("hstu_outproj_ln_bwd")(
        g8.data_ptr(), g8.stride(0), gs.data_ptr(), w8.data_ptr(), w8.stride(0), ws_.data_ptr(), x.data_ptr(),
        x.stride(0), u.data_ptr(), u.stride(0), w.data_ptr(), b.data_ptr(), pd, mean.contiguous().data_ptr(),
        rstd.contiguous().data_ptr(), N, D, _ACT[act], int(bool(silu_u)), float(dropout_ratio), _lib.ptr(mask),
        0 if mask is None else mask.stride(0), dx.data_ptr(), dx.stride(0), du.data_ptr(), du.stride(0),
        dw.data_ptr(), db.data_ptr(), ws.data_ptr(), nbytes, _stream(x))
    _lib.check(st, "hstu_outproj_ln_bwd")
    return dx, du, dw, db


def triton_layer_norm_mul_dropout_bwd(
    dy: torch.Tensor,
    x: torch.Tensor,
    u: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor,
    mean: torch.Tensor,
    rstd: torch.Tensor,
    BLOCK_D: int,
    num_warps: int,
    eps: float,
    training: bool,
    dropout_ratio: float,
    seed: Optional[int] = None,
    silu_u: bool = False,
    concat_u: bool = False,
    concat_x: bool = False,
    mul_u_activation_type: str = "none",
    compute_y: bool = False,
    random_mask: Optional[torch.Tensor] = None,
    du_row_width: int = 0,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
    """(dx, du, dweight, dbias, y); dweight / dbias in weight's dtype, y the
    recomputed bf16 forward output when ``compute_y``.  Without
    ``random_mask`` a training call redraws the mask from ``seed``."""
    mask = None
    if training and dropout_ratio > 0.0:
        mask = random_mask
        if mask is None:
            if seed is None:
                raise ValueError("training backward without random_mask needs the forward's seed")
            mask = create_dropout_mask(x.shape[0], x.shape[1], concat_u, concat_x, dropout_ratio, seed, x.device)
    dx, du, dw, db, y = _ln_bwd(dy, x, u, weight, bias, mean, rstd, dropout_ratio, mask, silu_u, concat_u,
                                concat_x, mul_u_activation_type, compute_y, du_row_width)
    return dx, du, dw.to(weight.dtype), db.to(bias.dtype), y


class LayerNormMulDropoutFunction(torch.autograd.Function):
    """Autograd of LN * U * dropout (``triton_hstu_linear.py:3953-4058``)."""

    @staticmethod
    def forward(ctx, x, u, weight, bias, eps, dropout_ratio, training, silu_u=False, concat_ux=False, seed=None,
                mul_u_activation_type="none"):
        if dropout_ratio == 0.0:
            training = False
        y, mean, rstd, _, _, seed, mask = triton_layer_norm_mul_dropout_fwd(
            x, u, weight, bias, eps, dropout_ratio, training, silu_u, concat_ux, concat_ux,
            mul_u_activation_type, seed)
        saved = [x, u, weight, bias, mean, rstd]
        if mask is not None:
            saved.append(mask)
        ctx.save_for_backward(*saved)
        ctx.has_mask = mask is not None
        ctx.cfg = (eps, dropout_ratio, training, silu_u, concat_ux, seed, mul_u_activation_type)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, u, weight, bias, mean, rstd = ctx.saved_tensors[:6]
        mask = ctx.saved_tensors[6] if ctx.has_mask else None
        eps, ratio, training, silu_u, concat_ux, seed, act = ctx.cfg
        dx, du, dw, db, _ = triton_layer_norm_mul_dropout_bwd(
            dy, x, u, weight, bias, mean, rstd, 0, 0, eps, training, ratio, seed, silu_u, concat_ux, concat_ux, act,
            False, mask)
        return dx, du, dw, db, None, None, None, None, None, None, None


def triton_norm_mul_dropout(
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
    group_norm: bool = False,
    num_heads: int = 1,
    linear_dim: int = -1,
    seed: Optional[int] = None,
) -> torch.Tensor:
    """Differentiable LN * U * dropout (``triton_hstu_linear.py:6446-6491``;
    like the reference, the concat is on only when both concat flags are)."""
    if group_norm:
        raise NotImplementedError("group norm is not served by this build")
    return LayerNormMulDropoutFunction.apply(x, u, weight, bias, eps, dropout_ratio, training, silu_u,
                                             concat_u and concat_x, seed)


# ---------------------------------------------------------------------------
# output block: LN * U * dropout -> output projection + residual
# ---------------------------------------------------------------------------
class ResidualLink:
    """Hands the output block's residual gradient of the layer input x to the
    preprocess backward of the same layer, which adds it inside its LayerNorm
    backward (dx = dres + LN backward, one rounding) instead of autograd adding
    the two bf16 gradients in a separate kernel.  The output block's backward
    runs first (its inputs are the preprocess outputs); it stores the gradient
    and returns None for x.

    The preprocess forward binds its x (``bind``); the output block uses the
    link only when its own residual input is that same tensor at the same
    version (``bound_to``), else it returns the residual gradient itself."""

    def __init__(self) -> None:
        self.grad: Optional[torch.Tensor] = None
        self._x: Optional["weakref.ref"] = None
        self._x_version = -1

    def bind(self, x: torch.Tensor) -> None:
        self._x = weakref.ref(x)
        self._x_version = x._version

    def bound_to(self, x: torch.Tensor) -> bool:
        return self._x is not None and self._x() is x and x._version == self._x_version

    def take(self) -> Optional[torch.Tensor]:
        g, self.grad = self.grad, None
        return g


class HSTUComputeOutputFunction(torch.autograd.Function):
    """``HSTUComputeOutputFunction`` (``triton_hstu_linear.py:5109-5900``),
    default (unfused-backward) contract: e4m3 LN output into the FP8 output
    projection when ``fp8_output_scale`` is given and y is recomputed in the
    backward, bf16 otherwise; backward = dgrad (bf16, or e5m2 x e4m3 FP8 with
    ``DLRM_HSTU_FP8_BWD=1`` once its scale is calibrated), the LN * U *
    dropout backward (recomputing y), bf16 wgrad."""

    @staticmethod
    def forward(ctx, attn, u, x, norm_weight, norm_bias, output_weight, eps, dropout_ratio, training,
                silu_u=False, concat_u=False, concat_x=False, mul_u_activation_type="none", group_norm=False,
                num_heads=1, linear_dim=-1, seed=None, recompute_y_in_backward=False, rng_row_indices=None,
                fp8_output_scale=None, fp8_backward=None, dropout_mask16=None, residual_link=None):
        if group_norm:
            raise NotImplementedError("group norm is not served by this build")
        if rng_row_indices is not None:
            raise NotImplementedError("rng_row_indices (compact rows) is not served")
        if dropout_ratio == 0.0:
            training = False
        # the scale is used once ready (a plain scale, or a calibrated state
        # buffer); until then the call runs bf16 and calibrates the state
        # (triton_hstu_linear.py:5260-5280).  It stays on the device.
        ready = _fp8.scale_ready(fp8_output_scale)
        use_fp8 = ready and recompute_y_in_backward
        seed = _seed(seed, training)
        scale = None
        if use_fp8:
            scale = _fp8.fp8_scale_tensor(fp8_output_scale).reshape(1)
            y, mean, rstd, mask = _ln_fwd(attn, u, norm_weight, norm_bias, eps, dropout_ratio, training, silu_u,
                                          concat_u, concat_x, mul_u_activation_type, seed, True, 1.0, out_scale=scale,
                                          mask16=dropout_mask16)
            out = _fp8.scaled_addmm_fp8_preq(y, scale, output_weight, x, out_dtype=x.dtype)
        else:
            y, mean, rstd, mask = _ln_fwd(attn, u, norm_weight, norm_bias, eps, dropout_ratio, training, silu_u,
                                          concat_u, concat_x, mul_u_activation_type, seed, False, 1.0,
                                          mask16=dropout_mask16)
            if fp8_output_scale is not None and not ready:
                _fp8.calibrate_scale_buffer(fp8_output_scale, y)
            out = _fp8.proj_mm(y, output_weight.to(y.dtype).t(), residual=x)
        saved = [attn, u, norm_weight, norm_bias, mean, rstd, output_weight]
        if not recompute_y_in_backward:
            saved.append(y)
        if mask is not None:
            saved.append(mask)
        # the e4m3 y feeds the FP8 output-projection weight gradient
        ctx.y8_scale = scale if (use_fp8 and bwd_fp8.out_wgrad_fp8(fp8_backward)) else None
        ctx.fp8_backward = fp8_backward
        if ctx.y8_scale is not None:
            saved.append(y)
        ctx.save_for_backward(*saved)
        ctx.recompute = bool(recompute_y_in_backward)
        ctx.has_mask = mask is not None
        # the preprocess forward tags u with its d(uvqk) row width: du is then
        # written as the leading columns of that buffer (triton_hstu_linear.py:5347-5350)
        ctx.du_row_width = int(getattr(u, "_hstu_duvqk_width", 0))
        ctx.cfg = (dropout_ratio, silu_u, concat_u, concat_x, mul_u_activation_type)
        # the link is used only for the x its preprocess forward was given
        ctx.residual_link = residual_link if residual_link is not None and residual_link.bound_to(x) else None
        return out

    @staticmethod
    def backward(ctx, dout):
        attn, u, norm_weight, norm_bias, mean, rstd, output_weight = ctx.saved_tensors[:7]
        i = 7
        y = None
        if not ctx.recompute:
            y = ctx.saved_tensors[i]
            i += 1
        mask = ctx.saved_tensors[i] if ctx.has_mask else None
        i += int(ctx.has_mask)
        y8 = ctx.saved_tensors[i] if ctx.y8_scale is not None else None
        ratio, silu_u, concat_u, concat_x, act = ctx.cfg
        dout = dout.contiguous()
        # the residual gradient of x: to the same layer's preprocess backward
        # when linked, else returned here
        dres_x = dout
        if ctx.residual_link is not None and ctx.needs_input_grad[2]:
            ctx.residual_link.grad = dout
            dres_x = None
        # FP8 dgrad (DLRM_HSTU_FP8_BWD=1; triton_hstu_linear.py:5586-5588): None
        # while the gradient's scale warms up, then e5m2 dout . e4m3 W^T
        cfg = ctx.fp8_backward
        # the fused FP8 dgrad + LN * U * dropout backward (dy never in HBM) when
        # the FP8 weight gradient needs no recomputed y and the shapes are the
        # kernel's ([u' | x | y] concat, D = 512)
        if (y8 is not None and bwd_fp8.enabled(cfg) and bwd_fp8.resolve(cfg).outproj_lnmd_fused and concat_u
                and concat_x and attn.shape[-1] == 512 and tuple(output_weight.shape) == (1536, 512)):
            ops = bwd_fp8.output_projection_dgrad_operands(dout, output_weight, snapshot_decode_scale=True,
                                                           config=cfg)
            if ops is not None:
                g8, gs, w8, ws = ops
                dattn, du, dw, db = _outproj_ln_bwd(g8, gs, w8, ws, attn, u, norm_weight, norm_bias, mean, rstd,
                                                    ratio, mask, silu_u, act, ctx.du_row_width)
                d_out_w = fp8_wgrad(y8, g8, ctx.y8_scale, gs).to(output_weight.dtype)
                return (dattn, du, dres_x, dw.to(norm_weight.dtype), db.to(norm_bias.dtype), d_out_w,
                        None, None, None, None, None, None, None, None, None, None, None, None, None, None, None,
                        None, None)
            # the gradient's scale warms up (this call is counted): bf16 dgrad
            q = None
        else:
            q = (bwd_fp8.output_projection_dgrad(dout, output_weight, return_quantized=True, config=cfg)
                 if bwd_fp8.enabled(cfg) else None)
        dy = q[0] if q is not None else _fp8.proj_mm(dout, output_weight)
        # FP8 weight gradient (DLRM_HSTU_FP8_BWD_OUT_WGRAD=1) from the forward's
        # e4m3 y and the dgrad's e5m2 dout: the bf16 y is then not recomputed
        fp8_w = y8 is not None and q is not None
        dattn, du, dw, db, y_re = _ln_bwd(dy, attn, u, norm_weight, norm_bias, mean, rstd, ratio, mask, silu_u,
                                          concat_u, concat_x, act, ctx.recompute and not fp8_w, ctx.du_row_width)
        if fp8_w:
            d_out_w = fp8_wgrad(y8, q[1], ctx.y8_scale, q[2]).to(output_weight.dtype)
        else:
            if y is None:
                y = y_re
            # y^T dout over the tokens: the split-K wgrad kernel
            d_out_w = token_wgrad(y, dout).to(output_weight.dtype)
        return (dattn, du, dres_x, dw.to(norm_weight.dtype), db.to(norm_bias.dtype), d_out_w,
                None, None, None, None, None, None, None, None, None, None, None, None, None, None, None, None, None)


def triton_hstu_compute_output(
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
    seed: Optional[int] = None,
    recompute_y_in_backward: bool = False,
    rng_row_indices: Optional[torch.Tensor] = None,
    fp8_output_scale: Optional[torch.Tensor] = None,
    *,
    fp8_backward: Optional[bwd_fp8.Fp8BackwardConfig] = None,
    dropout_mask16: Optional[bool] = None,
    residual_link: Optional[ResidualLink] = None,
) -> torch.Tensor:
    """x + dropout([u' | attn | m(u) * LN(attn)]) @ output_weight
    (``triton_hstu_linear.py:6494-6572``).  ``fp8_output_scale``: a
    one-element device scale, or the reference's [2 + steps] scale state
    (calibrated by the bf16 calls until frozen).  ``fp8_backward``: the FP8
    backward arm's settings, ``dropout_mask16`` the dropout mask scheme
    (default for both: the process default); ``residual_link`` hands x's
    residual gradient to the same layer's preprocess backward."""
    return HSTUComputeOutputFunction.apply(attn, u, x, norm_weight, norm_bias, output_weight, eps, dropout_ratio,
                                           training, silu_u, concat_u, concat_x, mul_u_activation_type, group_norm,
                                           num_heads, linear_dim, seed, recompute_y_in_backward, rng_row_indices,
                                           fp8_output_scale, fp8_backward, dropout_mask16, residual_link)


def hstu_compute_output(
    attn: torch.Tensor,
    u: torch.Tensor,
    x: torch.Tensor,
    norm_weight: torch.Tensor,
    norm_bias: torch.Tensor,
    norm_eps: float,
    output_weight: torch.Tensor,
    num_heads: int,
    linear_dim: int,
    dropout_ratio: float,
    training: bool,
    concat_u: bool,
    concat_x: bool,
    mul_u_activation_type: str,
    group_norm: bool,
    recompute_y_in_backward: bool,
    kernel: HammerKernel = HammerKernel.PYTORCH,
    rng_row_indices: Optional[torch.Tensor] = None,
    fp8_output_scale: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Layer-level dispatch (``ops/hstu_compute.py:147-215``): silu_u follows
    ``mul_u_activation_type == "silu"``; TRITON / HIP select the HIP kernels."""
    silu_u = mul_u_activation_type == "silu"
    if kernel in (HammerKernel.TRITON, HammerKernel.HIP):
        return triton_hstu_compute_output(attn, u, x, norm_weight, norm_bias, output_weight, norm_eps,
                                          dropout_ratio, training, silu_u, concat_u, concat_x,
                                          mul_u_activation_type, group_norm, num_heads, linear_dim, None,
                                          recompute_y_in_backward, rng_row_indices, fp8_output_scale)
    return pytorch_hstu_compute_output(attn, u, x, norm_weight, norm_bias, output_weight, norm_eps, dropout_ratio,
                                       training, silu_u, concat_u, concat_x, mul_u_activation_type, group_norm,
                                       num_heads, linear_dim)


# ---------------------------------------------------------------------------
# weighted LayerNorm (the UVQK GEMM's producer)
# ---------------------------------------------------------------------------
def triton_weighted_layer_norm_fwd(
    x: torch.Tensor,
    weight: Optional[torch.Tensor],
    bias: Optional[torch.Tensor],
    eps: float,
    mean: Optional[torch.Tensor] = None,
    rstd: Optional[torch.Tensor] = None,
    output_fp8: bool = False,
    inv_scale: float = 1.0,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(y, mean, rstd); y = LN(x) * weight + bias in bf16, or
    e4m3(clamp(y * inv_scale, +-448)) with ``output_fp8``
    (``ops/triton/triton_layer_norm.py:1668-1740``)."""
    if mean is not None or rstd is not None:
        raise NotImplementedError("precomputed mean / rstd are not served")
    if output_fp8 and weight is None:
        raise AssertionError("FP8 LayerNorm output requires learnable affine parameters")
    y, mean, rstd, _ = _ln_fwd(x, None, weight, bias, eps, 0.0, False, False, False, False, "none", 0, output_fp8,
                               inv_scale)
    return y, mean, rstd


def triton_weighted_layer_norm_bwd(
    dy: torch.Tensor,
    x: torch.Tensor,
    weight: Optional[torch.Tensor],
    bias: Optional[torch.Tensor],
    mean: torch.Tensor,
    rstd: torch.Tensor,
    learnable: bool,
    eps: float,
    BLOCK_D: int,
    residual: Optional[torch.Tensor] = None,
    dropout_mask: Optional[torch.Tensor] = None,
    dropout_scale: float = 1.0,
) -> Tuple[torch.Tensor, Optional[torch.Tensor], Optional[torch.Tensor]]:
    """(dx, dweight, dbias) (``ops/triton/triton_layer_norm.py:3574-3640``);
    dweight / dbias are None when not ``learnable``."""
    if residual is not None or dropout_mask is not None:
        raise NotImplementedError("residual / dropout-mask folds are not served")
    dx, _, dw, db, _ = _ln_bwd(dy, x, None, weight, bias, mean, rstd, 0.0, None, False, False, False, "none", False)
    if not learnable:
        return dx, None, None
    return dx, dw.to(weight.dtype), db.to(bias.dtype)
