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
