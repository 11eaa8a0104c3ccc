"""FP8 backward projection GEMMs: the e5m2-gradient dgrads of the output and
UVQK projections and their delayed-scale controller, on this build's kernels
(``hstu_cast_fp8_amax``, ``hstu_cast_fp8_amax_colsum``, ``hstu_fp8_gemm`` with
an e5m2 A operand).

Mirrors ``ops/triton/bwd_fp8.py`` (reference paths relative to
``recommendation_v4/hstu/generative_recommenders/``):

* ``quantize_row_major``        <- ``:827-866`` (one pass: cast at a device-side
  inverse scale, clamp to the format's max, and the input's amax)
* ``quantize_amax_colsum``      <- ``:378-434, 608-692`` (the same cast plus the
  fp32 column sums of the input, zero rows past M up to ``pad_to``)
* ``SiteScale``                 <- ``_SiteScale`` ``:869-1003`` (scale published
  from the window amax times MARGIN / FP8_MAX, refreshed every REFRESH_CALLS)
* ``quantize_gradient``         <- ``:1073-1154`` (None while warming up: the
  caller runs bf16)
* ``quantize_weight``           <- ``:1157-1189`` (e4m3 at unit margin)
* ``output_projection_dgrad``   <- ``:1347-1395`` (dY_e5m2 . W_e4m3^T, bf16 out)
* ``uvqk_projection_backward``  <- ``:2313-2520`` (dZ_e5m2 . W_e4m3^T dgrad, bf16
  wgrad or with ``DLRM_HSTU_FP8_BWD_UVQK_WGRAD=fp8t`` the e4m3 x e5m2 wgrad,
  the cast's column sum as the bias gradient)

Switches (the reference's names): ``DLRM_HSTU_FP8_BWD=1`` enables the path;
``DLRM_HSTU_FP8_BWD_MARGIN`` (8), ``_REFRESH_CALLS`` (200), ``_WARMUP_CALLS``
(4), ``_GRAD_FORMAT`` (e5m2 | e4m3); ``DLRM_HSTU_FP8_BWD_UVQK=1`` (with the
e5m2 format) enables the UVQK backward on its own, as in the reference.  They
are read when a call needs them, so a process can switch the path on and off.
"""

from __future__ import annotations

import os
from typing import Callable, Dict, Optional, Tuple

import torch

from . import _lib
from .wgrad import fp8_wgrad, token_wgrad

E4M3 = torch.float8_e4m3fn
E5M2 = torch.float8_e5m2
E4M3_MAX = 448.0
E5M2_MAX = 57344.0


def enabled() -> bool:
    return os.environ.get("DLRM_HSTU_FP8_BWD", "0") == "1"


def _margin() -> float:
    return float(os.environ.get("DLRM_HSTU_FP8_BWD_MARGIN", "8"))


def _refresh_calls() -> int:
    return max(1, int(os.environ.get("DLRM_HSTU_FP8_BWD_REFRESH_CALLS", "200")))


def _warmup_calls() -> int:
    return max(1, int(os.environ.get("DLRM_HSTU_FP8_BWD_WARMUP_CALLS", "4")))


def grad_dtype_and_limit() -> Tuple[torch.dtype, float]:
    fmt = os.environ.get("DLRM_HSTU_FP8_BWD_GRAD_FORMAT", "e5m2").lower()
    if fmt not in ("e5m2", "e4m3"):
        raise ValueError(f"DLRM_HSTU_FP8_BWD_GRAD_FORMAT={fmt!r}")
    return (E4M3, E4M3_MAX) if fmt == "e4m3" else (E5M2, E5M2_MAX)


def _code(dtype: torch.dtype) -> int:
    return {torch.bfloat16: _lib.HSTU_DTYPE_BF16, torch.float32: _lib.HSTU_DTYPE_FP32, E4M3: _lib.HSTU_DTYPE_FP8_E4M3,
            E5M2: _lib.HSTU_DTYPE_FP8_E5M2}[dtype]


def quantize_row_major(value: torch.Tensor, inv_scale: torch.Tensor, dtype: Optional[torch.dtype] = None,
                       limit: Optional[float] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """(fp8(clamp(value * inv_scale, +-limit)), amax(|value|)) in one pass;
    the amax is of the input, before scaling."""
    gdt, glim = grad_dtype_and_limit()
    dtype = gdt if dtype is None else dtype
    limit = glim if limit is None else limit
    src = value.detach()
    if src.dtype not in (torch.bfloat16, torch.float32):
        src = src.float()
    if not src.is_contiguous() or src.data_ptr() % 16:
        src = src.contiguous()
    n = src.numel()
    out = torch.empty(src.shape, dtype=dtype, device=src.device)
    if n % 32:
        raise NotImplementedError("the FP8 cast takes a multiple of 32 elements")
    parts = int(_lib.fn("hstu_cast_fp8_amax_partials")(n))
    partial = torch.empty(max(parts, 1), dtype=torch.float32, device=src.device)
    if n == 0:
        return out, torch.zeros((), dtype=torch.float32, device=src.device)
    inv = inv_scale.to(torch.float32).reshape(-1)[:1].contiguous()
    st = _lib.fn("hstu_cast_fp8_amax")(
        _code(src.dtype), src.data_ptr(), n, inv.data_ptr(), _code(dtype), float(limit), out.data_ptr(),
        partial.data_ptr(), parts, torch.cuda.current_stream(src.device).cuda_stream)
    _lib.check(st, "hstu_cast_fp8_amax")
    return out, partial[:parts].amax()


def quantize_amax_colsum(value: torch.Tensor, inv_scale: torch.Tensor, pad_to: int = 1,
                         out: Optional[torch.Tensor] = None,
                         dtype: Optional[torch.dtype] = None) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """One read of a row-major bf16 [M, N] gradient -> (fp8 copy [Mp, N], amax,
    colsum fp32 [N]); Mp = roundup(M, pad_to), rows >= M zero.  ``colsum`` is
    the sum over rows of the unquantized input (the bias gradient), in a fixed
    fp32 order (512-row stripes, then the stripes).  ``out``, if given, is a
    contiguous [Mp' >= M, N] tensor of the gradient format, filled the same
    way.  N % 256 == 0."""
    dtype = grad_dtype_and_limit()[0] if dtype is None else dtype
    limit = E4M3_MAX if dtype == E4M3 else E5M2_MAX
    if value.dim() != 2 or value.dtype != torch.bfloat16:
        raise ValueError("quantize_amax_colsum takes a 2-D bf16 gradient")
    src = value.detach()
    if src.stride(1) != 1 or src.stride(0) % 8 or src.data_ptr() % 16:
        src = src.contiguous()
    m, n = src.shape
    if out is None:
        if pad_to < 1:
            raise ValueError("pad_to >= 1")
        out = torch.empty(((m + pad_to - 1) // pad_to * pad_to, n), dtype=dtype, device=src.device)
    elif (out.dim() != 2 or not out.is_contiguous() or out.dtype != dtype or out.shape[1] != n or out.shape[0] < m
          or out.device != src.device):
        raise ValueError("out must be a contiguous [>= M, N] tensor of the gradient format")
    ws_bytes = int(_lib.fn("hstu_cast_fp8_amax_colsum_workspace_bytes")(m, n))
    if ws_bytes < 0:
        raise NotImplementedError("the column-sum cast takes N % 256 == 0")
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=src.device)
    colsum = torch.empty(n, dtype=torch.float32, device=src.device)
    amax = torch.empty((), dtype=torch.float32, device=src.device)
    inv = inv_scale.to(torch.float32).reshape(-1)[:1].contiguous()
    st = _lib.fn("hstu_cast_fp8_amax_colsum")(
        src.data_ptr(), src.stride(0), m, n, inv.data_ptr(), _code(dtype), float(limit), out.data_ptr(),
        out.shape[0], colsum.data_ptr(), amax.data_ptr(), ws.data_ptr(), ws_bytes,
        torch.cuda.current_stream(src.device).cuda_stream)
    _lib.check(st, "hstu_cast_fp8_amax_colsum")
    return out, amax, colsum


class SiteScale:
    """One backward tensor's scale, held and published on the device.

    ``scale`` dequantizes (fp8 value * scale = original), ``inv_scale`` is what
    the cast multiplies by.  The window's amax accumulates in ``pending``.
    """

    def __init__(self, site: str, device: torch.device) -> None:
        self.site = site
        self.calls = 0
        self.scale = torch.zeros(1, dtype=torch.float32, device=device)
        self.inv_scale = torch.zeros(1, dtype=torch.float32, device=device)
        self.pending = torch.zeros((), dtype=torch.float32, device=device)
        self.clipped_windows = torch.zeros((), dtype=torch.int64, device=device)
        self.published = False

    def accumulate(self, amax: torch.Tensor) -> None:
        torch.maximum(self.pending, amax, out=self.pending)

    def publish(self) -> None:
        """The window's amax becomes the next window's scale (clamped away
        from zero so an all-zero window cannot publish an infinite inverse)."""
        _, limit = grad_dtype_and_limit()
        self.scale.copy_((self.pending.clamp_min(1.0e-30) * (_margin() / limit)).reshape(1))
        self.inv_scale.copy_(1.0 / self.scale)
        self.pending.zero_()
        self.published = True

    def note_clipping(self, amax: torch.Tensor) -> None:
        _, limit = grad_dtype_and_limit()
        self.clipped_windows += (amax > self.scale.reshape(()) * limit).to(torch.int64)


_sites: Dict[str, SiteScale] = {}
_layer_index: Dict[Tuple[str, int], int] = {}


def reset_sites() -> None:
    """Forget every site's state (tests, or a new run in the same process)."""
    _sites.clear()
    _layer_index.clear()


def site_name(site: str, discriminator: Optional[int]) -> str:
    """One layer's instance of a site, indexed in order of first appearance."""
    if discriminator is None:
        return site
    key = (site, discriminator)
    if key not in _layer_index:
        _layer_index[key] = sum(1 for k in _layer_index if k[0] == site)
    return f"{site}.L{_layer_index[key]}"


def site_state(site: str, device: torch.device) -> SiteScale:
    st = _sites.get(site)
    if st is None:
        st = _sites[site] = SiteScale(site, device)
    return st


def quantize_gradient(site: str, gradient: torch.Tensor, discriminator: Optional[int] = None,
                      snapshot_decode_scale: bool = False) -> Optional[Tuple[torch.Tensor, torch.Tensor]]:
    """(fp8 gradient, dequantization scale) under the delayed-scale policy, or
    None while the site warms up (the caller's signal to run bf16).

    As in the reference, the returned scale is the site's scale tensor, which
    a refresh on this call has already updated in place; with
    ``snapshot_decode_scale`` it is a copy of the scale the payload was cast
    with, taken before the refresh."""
    if not enabled():
        return None
    if gradient.numel() == 0 or gradient.dtype not in (torch.bfloat16, torch.float32, torch.float16):
        return None
    state = site_state(site_name(site, discriminator), gradient.device)
    state.calls += 1
    if not state.published:
        state.accumulate(gradient.detach().abs().amax().float())
        if state.calls >= _warmup_calls():
            state.publish()
        return None
    q, amax = quantize_row_major(gradient, state.inv_scale)
    state.note_clipping(amax)
    state.accumulate(amax)
    decode = state.scale.clone() if snapshot_decode_scale else state.scale
    if state.calls % _refresh_calls() == 0:
        state.publish()
    return q, decode


def quantize_weight(weight: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """e4m3 at unit margin: scale = amax / 448 on the device, cast at 1 / scale."""
    amax = weight.detach().abs().amax().float().clamp_min(1.0e-30)
    scale = (amax / E4M3_MAX).reshape(1)
    q, _ = quantize_row_major(weight, 1.0 / scale, dtype=E4M3, limit=E4M3_MAX)
    return q, scale


def _has_stable_identity(weight: torch.Tensor) -> bool:
    return weight.is_leaf and weight.requires_grad


def fp8_dgrad(grad8: torch.Tensor, grad_scale: torch.Tensor, w8: torch.Tensor, w_scale: torch.Tensor,
              out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """grad8 [M, K] (e5m2 or e4m3) . w8 [N, K]^T (e4m3) * grad_scale * w_scale -> bf16 [M, N]."""
    if out_dtype != torch.bfloat16:
        raise NotImplementedError("the FP8 dgrad writes bf16")
    M, K = grad8.shape
    N = w8.shape[0]
    if w8.shape[1] != K or w8.dtype != E4M3:
        raise ValueError("w8 must be e4m3 [N, K]")
    g = grad8.contiguous()
    w = w8.contiguous()
    sa = grad_scale.to(torch.float32).reshape(-1)[:1].contiguous()
    sb = w_scale.to(torch.float32).reshape(-1)[:1].contiguous()
    out = torch.empty((M, N), dtype=torch.bfloat16, device=g.device)
    if M == 0:
        return out
    st = _lib.fn("hstu_fp8_gemm")(
        _code(g.dtype), g.data_ptr(), K, w.data_ptr(), K, sa.data_ptr(), 0, sb.data_ptr(), 0, None, None, 0,
        out.data_ptr(), N, _lib.HSTU_DTYPE_BF16, None, M, N, K, 0, 0, torch.cuda.current_stream(g.device).cuda_stream)
    _lib.check(st, "hstu_fp8_gemm")
    return out


def out_wgrad_fp8() -> bool:
    """``DLRM_HSTU_FP8_BWD_OUT_WGRAD=1`` (with the FP8 backward on): the output
    projection's weight gradient from the forward's e4m3 LN * U output and the
    dgrad's e5m2 dout cast (``triton_hstu_linear.py:87-110``)."""
    return enabled() and os.environ.get("DLRM_HSTU_FP8_BWD_OUT_WGRAD", "0") == "1"


def output_projection_dgrad(gradient: torch.Tensor, weight: torch.Tensor, return_quantized: bool = False):
    """``dy = gradient @ weight^T`` in FP8 (gradient [M, N_out], weight
    [K_in, N_out] as stored by the layer), or None to fall back to bf16.
    With ``return_quantized``: (dy, gradient_fp8, its decode scale), for a
    weight gradient that reuses the cast."""
    if not enabled() or not _has_stable_identity(weight):
        return None
    if gradient.dim() != 2 or gradient.shape[-1] % 128 or weight.shape[0] % 128:
        return None
    quantized = quantize_gradient("output_projection", gradient, discriminator=weight.data_ptr())
    if quantized is None:
        return None
    g8, gs = quantized
    w8, ws = quantize_weight(weight)
    dy = fp8_dgrad(g8, gs, w8, ws, gradient.dtype if gradient.dtype == torch.bfloat16 else torch.bfloat16)
    return (dy, g8, gs) if return_quantized else dy


def uvqk_fp8_backward_enabled() -> bool:
    """``DLRM_HSTU_FP8_BWD_UVQK=1`` with the e5m2 gradient format."""
    return (os.environ.get("DLRM_HSTU_FP8_BWD_UVQK", "0") == "1"
            and grad_dtype_and_limit()[0] == E5M2)


def uvqk_wgrad_fp8t() -> bool:
    """``DLRM_HSTU_FP8_BWD_UVQK_WGRAD=fp8t`` (with the UVQK arm on): the UVQK
    weight gradient from the forward's e4m3 LN output and the e5m2 gradient
    (``uvqk_wgrad_fp8t``, ``ops/triton/bwd_fp8.py:1755-1762``)."""
    return (uvqk_fp8_backward_enabled()
            and os.environ.get("DLRM_HSTU_FP8_BWD_UVQK_WGRAD", "bf16").strip().lower() == "fp8t")


def uvqk_projection_backward(
    dz: Optional[torch.Tensor],
    normed_x: Optional[torch.Tensor],
    input_scale_value: Optional[float],
    weight: torch.Tensor,
    site: str = "uvqk_projection",
    per_layer: bool = True,
    normed_x_fp8_t: Optional[torch.Tensor] = None,
    recompute_normed_x: Optional[Callable[[], torch.Tensor]] = None,
) -> Optional[Tuple[torch.Tensor, torch.Tensor, torch.Tensor]]:
    """(d_normed_x, d_weight, d_bias fp32) of ``z = normed_x @ weight + b``
    with an FP8 dgrad, or None for the caller's bf16 path.

    dz [M, N] bf16 (N % 256 == 0), weight [K, N] as the layer stores it.  One
    cast of dz gives its e5m2 copy, amax and column sum (the bias gradient);
    the dgrad is dz_e5m2 . W_e4m3^T at the site's delayed scale (a snapshot
    of the scale the payload was cast with, on a refresh call); the weight
    gradient is the bf16 product normed_x^T dz (the split-K wgrad kernel).
    ``per_layer`` keys the scale on the weight's storage (then it must be the
    leaf parameter).
    ``normed_x`` may be None when ``recompute_normed_x`` is given.  With
    ``uvqk_wgrad_fp8t()``, ``normed_x_fp8_t`` (the forward's e4m3 LN output,
    here row-major [M, K] -- the kernel reads token rows directly, so no
    token-major copy is made) and ``input_scale_value`` > 0, the weight
    gradient is the FP8 product (x8 s_x)^T (dz8 s_dz) instead."""
    if not uvqk_fp8_backward_enabled():
        return None
    if per_layer and not _has_stable_identity(weight):
        return None
    if (dz is None or dz.dim() != 2 or not dz.is_contiguous() or dz.dtype != torch.bfloat16 or dz.shape[1] % 256
            or dz.shape[0] == 0 or weight.dim() != 2 or weight.shape[1] != dz.shape[1] or weight.shape[0] % 128
            or (normed_x is None and recompute_normed_x is None)
            or (normed_x is not None and tuple(normed_x.shape) != (dz.shape[0], weight.shape[0]))):
        return None
    state = site_state(site_name(site, weight.data_ptr() if per_layer else None), dz.device)
    state.calls += 1
    if not state.published:
        state.accumulate(dz.detach().abs().amax().float())
        if state.calls >= _warmup_calls():
            state.publish()
        return None
    dz8, amax, colsum = quantize_amax_colsum(dz, state.inv_scale, dtype=E5M2)
    state.note_clipping(amax)
    state.accumulate(amax)
    # the payload was cast with the scale in use now; a refresh rewrites it in place
    if state.calls % _refresh_calls() == 0:
        grad_scale = state.scale.clone()
        state.publish()
    else:
        grad_scale = state.scale
    w8, w_scale = quantize_weight(weight)
    use_tm = (uvqk_wgrad_fp8t() and normed_x_fp8_t is not None and input_scale_value is not None
              and input_scale_value > 0.0 and normed_x_fp8_t.dtype == E4M3
              and tuple(normed_x_fp8_t.shape) == (dz.shape[0], weight.shape[0]))
    if use_tm:
        sx = torch.full((1,), float(input_scale_value), dtype=torch.float32, device=dz.device)
        d_w = fp8_wgrad(normed_x_fp8_t, dz8, sx, grad_scale)
    else:
        xn = normed_x if normed_x is not None else recompute_normed_x()
        d_w = token_wgrad(xn, dz)
    d_x = fp8_dgrad(dz8, grad_scale, w8, w_scale)
    return d_x, d_w, colsum
