"""CPU restatement of the FP8 backward projection arm.

TEST INFRASTRUCTURE ONLY (imported by ``tests/`` and nowhere in the product).

Follows ``ops/triton/bwd_fp8.py`` (paths relative to
``recommendation_v4/hstu/generative_recommenders/``):

* ``cast_amax``        -- ``_quantize_amax_kernel`` / ``quantize_row_major``
  (:194-217, :827-866): fp8(clamp(x * inv_scale, +-limit)) and max |x|.
  The conversion is torch's round-to-nearest-even float8 cast (a library
  routine); the multiply is fp32 as in the kernel.  Pinned by the decode
  bound |fp8 * scale - x| <= half a step and by exact values at powers of two.
* ``published_scale``  -- ``_SiteScale.publish`` (:905-917):
  max(amax, 1e-30) * MARGIN / FP8_MAX.  Pinned by the closed form: the window
  amax lands at FP8_MAX / MARGIN after the cast.
* ``weight_scale``     -- ``quantize_weight`` (:1157-1189): amax / 448.
* ``dgrad``            -- ``output_projection_dgrad`` (:1347-1395): the fp64
  product of the dequantized operands, dY8 * s_dy . (W8 * s_w)^T.
* ``cast_amax_colsum`` -- ``_quantize_amax_colsum_kernel`` /
  ``quantize_amax_colsum`` (:378-434, :608-692): the ``cast_amax`` payload,
  rows M .. roundup(M, pad_to) zero, and the float64 column sums of the
  unquantized input.  Pinned by closed-form column sums (constant and
  alternating columns) and by the payload equal to ``cast_amax``'s.
* ``uvqk_backward``    -- ``uvqk_projection_backward`` (:2313-2520): dgrad of
  the dequantized operands, wgrad normed_x^T dz and the bias gradient
  colsum(dz), all float64.  Pinned through ``dgrad`` and
  ``cast_amax_colsum``, and by the unquantized case equal to
  ``torch.autograd`` of z = x W + b.
* ``wgrad``            -- ``fp8_wgrad`` / ``triton_addmm_bwd``'s dw
  (``ops/triton/fp8_wgrad.py:109-160``, ``ops/triton/triton_addmm.py:1737-1750``):
  (a sa)^T (b sb) over the token axis in float64.  Pinned by closed forms:
  all-ones a gives b's column sums, one-hot b rows pick a's rows.
"""

from __future__ import annotations

import torch


def cast_amax(x: torch.Tensor, inv_scale: float, dtype: torch.dtype, limit: float):
    xf = x.detach().float().cpu()
    inv = torch.tensor(inv_scale, dtype=torch.float32)
    q = (xf * inv).clamp(-limit, limit).to(dtype)
    return q, xf.abs().amax()


def published_scale(window_amax: float, margin: float, fp8_max: float) -> float:
    a = torch.tensor(window_amax, dtype=torch.float32).clamp_min(1.0e-30)
    return float(a * torch.tensor(margin / fp8_max, dtype=torch.float32))


def weight_scale(weight: torch.Tensor) -> torch.Tensor:
    amax = weight.detach().abs().amax().float().clamp_min(1.0e-30)
    return (amax / 448.0).reshape(1)


def dgrad(g8: torch.Tensor, g_scale: float, w8: torch.Tensor, w_scale: float) -> torch.Tensor:
    """g8 [M, K], w8 [N, K] (float8 tensors) -> float64 [M, N]."""
    return (g8.double() * g_scale) @ (w8.double() * w_scale).t()


def cast_amax_colsum(x: torch.Tensor, inv_scale: float, dtype: torch.dtype, limit: float, pad_to: int = 1):
    """x [M, N] -> (fp8 [roundup(M, pad_to), N], amax, float64 colsum [N])."""
    m, n = x.shape
    if m == 0:
        q, amax = torch.zeros((0, n), dtype=torch.uint8).view(dtype), torch.zeros(())
    else:
        q, amax = cast_amax(x, inv_scale, dtype, limit)
    mp = (m + pad_to - 1) // pad_to * pad_to
    out = torch.zeros((mp, n), dtype=torch.uint8).view(dtype)
    out[:m] = q
    return out, amax, x.detach().double().cpu().sum(0)


def uvqk_backward(dz: torch.Tensor, normed_x: torch.Tensor, dz8: torch.Tensor, g_scale: float,
                  w8: torch.Tensor, w_scale: float):
    """(d_normed_x, d_weight, d_bias) in float64: the FP8 dgrad of the
    dequantized operands (w8 [K, N] as the layer stores the weight), the
    wgrad normed_x^T dz and the column sum of dz."""
    d_x = dgrad(dz8, g_scale, w8, w_scale)
    d_w = normed_x.double().cpu().t() @ dz.double().cpu()
    return d_x, d_w, dz.double().cpu().sum(0)


def wgrad(a: torch.Tensor, b: torch.Tensor, scale_a: float = 1.0, scale_b: float = 1.0) -> torch.Tensor:
    """a [T, N1], b [T, N2] (any float dtype, fp8 included) -> float64 [N1, N2]."""
    return (a.double().cpu() * scale_a).t() @ (b.double().cpu() * scale_b)
