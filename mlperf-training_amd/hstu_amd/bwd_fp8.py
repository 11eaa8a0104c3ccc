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

Configuration is an explicit ``Fp8BackwardConfig`` passed by the caller
(``config=``) or the process default (``default_config()``), which is read
once from the reference's switch names -- ``DLRM_HSTU_FP8_BWD=1`` enables the
path; ``DLRM_HSTU_FP8_BWD_MARGIN`` (8), ``_REFRESH_CALLS`` (200),
``_WARMUP_CALLS`` (4), ``_GRAD_FORMAT`` (e5m2 | e4m3);
``DLRM_HSTU_FP8_BWD_UVQK=1`` (with the e5m2 format) enables the UVQK backward
on its own, as in the reference; ``_UVQK_WGRAD=fp8t`` and ``_OUT_WGRAD=1``
the FP8 weight gradients -- and can be replaced with ``set_default_config``.
No call reads the environment.
"""

from __future__ import annotations

import dataclasses
import os
from typing import Callable, Dict, Optional, Tuple

import torch

from . import _lib
from .wgrad import fp8_wgrad, token_wgrad

E4M3 = torch.float8_e4m3fn
E5M2 = torch.float8_e5m2
E4M3_MAX = 448.0
E5M2_MAX = 57344.0


@dataclasses.dataclass(frozen=True)
class Fp8BackwardConfig:
    """The FP8 backward arm's settings (the reference's switches, as values).

    enabled: the output-projection e5m2 dgrad (``DLRM_HSTU_FP8_BWD``);
    uvqk: the UVQK e5m2 dgrad (``DLRM_HSTU_FP8_BWD_UVQK``, e5m2 only);
    out_wgrad_fp8 / uvqk_wgrad_fp8t: the FP8 weight gradients;
    margin, warmup_calls, refresh_calls, grad_format: the delayed-scale policy;
    attn_full_fp8: the attention's full-FP8 backward (``DLRM_HSTU_FP8_BWD_FULL``;
    None: the attention op's process default);
    outproj_lnmd_fused: the output projection's e5m2 dgrad and the LN * U *
    dropout backward as one kernel when the FP8 weight gradient is on
    (``DLRM_HSTU_FP8_BWD_OUTPROJ_LNMD_FUSED``, ``triton_hstu_linear.py:5410-5470``);
    attn_ssc_k / attn_dsc_k: the full-FP8 attention backward's P and dS
    pre-scale exponents relative to ceil(log2 N)
    (``DLRM_HSTU_FP8_BWD_FULL_SSC_K`` / ``_DSC_K``, ``hstu_flydsl_mha.py:1351-1370``;
    None: the environment, read per call as the reference does; the
    production gin sets DSC_K = -5, ``yambda_5b.gin:3764-3799``).
    """

    enabled: bool = False
    uvqk: bool = False
    out_wgrad_fp8: bool = False
    uvqk_wgrad_fp8t: bool = False
    margin: float = 8.0
    warmup_calls: int = 4
    refresh_calls: int = 200
    grad_format: str = "e5m2"
    attn_full_fp8: Optional[bool] = None
    outproj_lnmd_fused: bool = False
    attn_ssc_k: Optional[int] = None
    attn_dsc_k: Optional[int] = None

    def __post_init__(self):
        if self.grad_format not in ("e5m2", "e4m3"):
            raise ValueError(f"grad_format {self.grad_format!r}: expected e5m2 | e4m3")
        if self.warmup_calls < 1 or self.refresh_calls < 1:
            raise ValueError("warmup_calls and refresh_calls must be >= 1")

    @classmethod
    def from_env(cls, env=None) -> "Fp8BackwardConfig":
        """The reference's switch names (``ops/triton/bwd_fp8.py``), read once."""
        env = os.environ if env is None else env
        return cls(
            enabled=env.get("DLRM_HSTU_FP8_BWD", "0") == "1",
            uvqk=env.get("DLRM_HSTU_FP8_BWD_UVQK", "0") == "1",
            out_wgrad_fp8=env.get("DLRM_HSTU_FP8_BWD_OUT_WGRAD", "0") == "1",
            uvqk_wgrad_fp8t=env.get("DLRM_HSTU_FP8_BWD_UVQK_WGRAD", "bf16").strip().lower() == "fp8t",
            margin=float(env.get("DLRM_HSTU_FP8_BWD_MARGIN", "8")),
            warmup_calls=max(1, int(env.get("DLRM_HSTU_FP8_BWD_WARMUP_CALLS", "4"))),
            refresh_calls=max(1, int(env.get("DLRM_HSTU_FP8_BWD_REFRESH_CALLS", "200"))),
            grad_format=env.get("DLRM_HSTU_FP8_BWD_GRAD_FORMAT", "e5m2").lower(),
            outproj_lnmd_fused=env.get("DLRM_HSTU_FP8_BWD_OUTPROJ_LNMD_FUSED", "0") == "1",
        )

    @property
    def grad_dtype(self) -> torch.dtype:
        return E4M3 if self.grad_format == "e4m3" else E5M2

    @property
    def grad_limit(self) -> float:
        return E4M3_MAX if self.grad_format == "e4m3" else E5M2_MAX


_default: Optional[Fp8BackwardConfig] = None


def default_config() -> Fp8BackwardConfig:
    """The process default: the environment's switches, read on first use."""
    global _default
    if _default is None:
        _default = Fp8BackwardConfig.from_env()
    return _default


def set_default_config(cfg: Optional[Fp8BackwardConfig]) -> None:
    """Replace the process default (None: read the environment again on next use)."""
    global _default
    _default = cfg


def resolve(config: Optional[Fp8BackwardConfig]) -> Fp8BackwardConfig:
    """``config``, or the process default when None."""
    return default_config() if config is None else config


def _cfg(config: Optional[Fp8BackwardConfig]) -> Fp8BackwardConfig:
    return default_config() if config is None else config


def enabled(config: Optional[Fp8BackwardConfig] = None) -> bool:
    return _cfg(config).enabled


def grad_dtype_and_limit(config: Optional[Fp8BackwardConfig] = None) -> Tuple[torch.dtype, float]:
    c = _cfg(config)
    return c.grad_dtype, c.grad_limit


def _code(dtype: torch.dtype) -> int:
    return {torch.bfloat16: _lib.HSTU_DTYPE_BF16, torch.float32: _lib.HSTU_DTYPE_FP32, E4M3: _lib.HSTU_DTYPE_FP8_E4M3,
            E5M2: _lib.HSTU_DTYPE_FP8_E5M2}[dtype]


def quantize_row_major(value: torch.Tensor, inv_scale: torch.Tensor, dtype: Optional[torch.dtype] = None,
                       limit: Optional[float] = None, partials: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """(fp8(clamp(value * inv_scale, +-limit)), amax(|value|)) in one pass;
    the amax is of the input, before scaling (with ``partials``, its
    per-8192-element block maxima instead, for ``GradScaleSite.update``).
    dtype / limit default to the process default's gradient format."""
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
        return out, torch.zeros(1 if partials else (), dtype=torch.float32, device=src.device)
    inv = inv_scale.to(torch.float32).reshape(-1)[:1].contiguous()
    st = _lib.fn("hstu_cast_fp8_amax")(
        _code(src.dtype), src.data_ptr(), n, inv.data_ptr(), _code(dtype), float(limit), out.data_ptr(),
        partial.data_ptr(), parts, torch.cuda.current_stream(src.device).cuda_stream)
    _lib.check(st, "hstu_cast_fp8_amax")
    return out, (partial[:parts] if partials else partial[:parts].amax())


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


class GradScaleSite:
    """Delayed scaling of one backward tensor (one site of one layer).

    All numbers live in one device tensor ``state`` = [scale, inverse scale,
    peak of the current window, windows whose amax overflowed the format], so
    publishing a scale is a device-side update with no host read.  ``scale``
    and ``inv_scale`` are views of it: the dequantization scale (fp8 value *
    scale = gradient) and what the cast multiplies by.  The host keeps only
    the call count.

    Policy (the reference's, ``ops/triton/bwd_fp8.py:869-1154``): the first
    ``warmup_calls`` calls are not quantized (the caller runs bf16) and only
    feed the window; then the window's peak times margin / format max becomes
    the scale, and every ``refresh_calls``-th call publishes the window that
    ends with it.
    """

    def __init__(self, device: torch.device) -> None:
        self.state = torch.zeros(4, dtype=torch.float32, device=device)
        self.calls = 0
        self.live = False

    @property
    def scale(self) -> torch.Tensor:
        return self.state[0:1]

    @property
    def inv_scale(self) -> torch.Tensor:
        return self.state[1:2]

    @property
    def overflow_windows(self) -> torch.Tensor:
        return self.state[3]

    def fold(self, amax: torch.Tensor, cfg: Fp8BackwardConfig) -> None:
        """Add one call's max |gradient| to the window (and, once quantizing,
        count the call if that amax overflowed the scale in use)."""
        a = amax.reshape(1).to(torch.float32)
        if self.live:
            self.state[3:4].add_((a > self.state[0:1] * cfg.grad_limit).to(torch.float32))
        torch.maximum(self.state[2:3], a, out=self.state[2:3])

    def roll(self, cfg: Fp8BackwardConfig) -> None:
        """Publish the window's scale and start a new window."""
        s = self.state[2:3].clamp_min(1.0e-30) * (cfg.margin / cfg.grad_limit)
        self.state[0:3].copy_(torch.cat([s, s.reciprocal(), torch.zeros_like(s)]))
        self.live = True

    def update(self, amax_values: torch.Tensor, cfg: Fp8BackwardConfig, roll: bool,
               snapshot: bool = False) -> Optional[torch.Tensor]:
        """``fold`` of the max of ``amax_values`` (a cast's per-block partials
        or one amax), then, with ``snapshot``, a copy of the scale in use, then
        ``roll`` when ``roll`` -- in one device launch (``hstu_fp8_site_update``),
        the same arithmetic as those methods.  Returns the snapshot."""
        vals = amax_values.reshape(-1)
        if not self.state.is_cuda:  # host tensors (the policy's CPU tests): the same steps in torch
            self.fold(vals.amax(), cfg)
            snap = self.scale.clone() if snapshot else None
            if roll:
                self.roll(cfg)
            return snap
        if vals.dtype != torch.float32 or not vals.is_contiguous():
            vals = vals.to(torch.float32).contiguous()
        snap = torch.empty(1, dtype=torch.float32, device=self.state.device) if snapshot else None
        st = _lib.fn("hstu_fp8_site_update")(
            vals.data_ptr(), vals.numel(), self.state.data_ptr(), float(cfg.grad_limit), int(self.live), int(roll),
            float(cfg.margin / cfg.grad_limit), _lib.ptr(snap), torch.cuda.current_stream(vals.device).cuda_stream)
        _lib.check(st, "hstu_fp8_site_update")
        if roll:
            self.live = True
        return snap

    def admit(self, cfg: Fp8BackwardConfig) -> Tuple[bool, bool]:
        """Count this call: (quantize it?, does it end a window?)."""
        self.calls += 1
        if not self.live:
            return False, self.calls >= cfg.warmup_calls
        return True, self.calls % cfg.refresh_calls == 0


class _Registry:
    """Sites by (name, layer).  A layer is numbered by the order in which its
    discriminator (the weight's storage address) first appears for a site."""

    def __init__(self) -> None:
        self.sites: Dict[Tuple[str, int], GradScaleSite] = {}
        self.layers: Dict[str, Dict[int, int]] = {}

    def layer_of(self, site: str, discriminator: Optional[int]) -> int:
        if discriminator is None:
            return -1
        seen = self.layers.setdefault(site, {})
        return seen.setdefault(discriminator, len(seen))

    def get(self, site: str, discriminator: Optional[int], device: torch.device) -> GradScaleSite:
        key = (site, self.layer_of(site, discriminator))
        found = self.sites.get(key)
        if found is None:
            found = self.sites[key] = GradScaleSite(device)
        return found


_registry = _Registry()


def reset_sites() -> None:
    """Forget every site's state (tests, or a new run in the same process)."""
    global _registry
    _registry = _Registry()


def site_name(site: str, discriminator: Optional[int]) -> str:
    """Printable name of one layer's instance of a site: ``site`` or ``site.L<n>``."""
    layer = _registry.layer_of(site, discriminator)
    return site if layer < 0 else f"{site}.L{layer}"


def find_site(site: str, discriminator: Optional[int] = None, layer: Optional[int] = None) -> Optional[GradScaleSite]:
    """The state of a site (by its discriminator, or by layer number), if it exists."""
    if layer is None:
        layer = -1 if discriminator is None else _registry.layers.get(site, {}).get(discriminator, -2)
    return _registry.sites.get((site, layer))


def quantize_gradient(site: str, gradient: torch.Tensor, discriminator: Optional[int] = None,
                      snapshot_decode_scale: bool = False,
                      config: Optional[Fp8BackwardConfig] = None) -> Optional[Tuple[torch.Tensor, torch.Tensor]]:
    """(fp8 gradient, dequantization scale) under the delayed-scale policy, or
    None while the site warms up (the caller's signal to run bf16).

    On a call that ends a window the site publishes a new scale in place
    after the cast.  The returned scale is then, as in the reference, the
    live (already refreshed) scale tensor, unless ``snapshot_decode_scale``
    asks for a copy of the scale the payload was cast with."""
    cfg = _cfg(config)
    if not cfg.enabled:
        return None
    if gradient.numel() == 0 or gradient.dtype not in (torch.bfloat16, torch.float32, torch.float16):
        return None
    ctl = _registry.get(site, discriminator, gradient.device)
    quantize, ends_window = ctl.admit(cfg)
    if not quantize:
        ctl.update(gradient.detach().abs().amax(), cfg, roll=ends_window)
        return None
    payload, partial = quantize_row_major(gradient, ctl.inv_scale, cfg.grad_dtype, cfg.grad_limit, partials=True)
    snap = ctl.update(partial, cfg, roll=ends_window, snapshot=ends_window and snapshot_decode_scale)
    return payload, (snap if snap is not None else ctl.scale)


def quantize_weight(weight: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """e4m3 at unit margin: scale = max(amax, 1e-30) / 448 on the device, cast
    at 1 / scale (``quantize_weight``, ``ops/triton/bwd_fp8.py:1157-1175``), in
    two launches (``hstu_quantize_e4m3_unit``; bitwise equal to the torch
    expression ``weight.abs().amax().float().clamp_min(1e-30) / 448``, which
    multiplies by fp32(1 / 448), and the cast at its reciprocal)."""
    src = weight.detach()
    if src.dtype not in (torch.bfloat16, torch.float32):
        src = src.float()
    if not src.is_contiguous() or src.data_ptr() % 16:
        src = src.contiguous()
    n = src.numel()
    if n == 0 or n % 32:
        amax = src.abs().amax().float().clamp_min(1.0e-30)
        scale = (amax / E4M3_MAX).reshape(1)
        q, _ = quantize_row_major(weight, 1.0 / scale, dtype=E4M3, limit=E4M3_MAX)
        return q, scale
    q = torch.empty(src.shape, dtype=E4M3, device=src.device)
    scale = torch.empty(1, dtype=torch.float32, device=src.device)
    parts = int(_lib.fn("hstu_cast_fp8_amax_partials")(n))
    partial = torch.empty(parts, dtype=torch.float32, device=src.device)
    st = _lib.fn("hstu_quantize_e4m3_unit")(
        _code(src.dtype), src.data_ptr(), n, q.data_ptr(), scale.data_ptr(), partial.data_ptr(), parts,
        torch.cuda.current_stream(src.device).cuda_stream)
    _lib.check(st, "hstu_quantize_e4m3_unit")
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


def out_wgrad_fp8(config: Optional[Fp8BackwardConfig] = None) -> bool:
    """The output projection's weight gradient in FP8, from the forward's e4m3
    LN * U output and the dgrad's e5m2 dout cast (``DLRM_HSTU_FP8_BWD_OUT_WGRAD``,
    ``triton_hstu_linear.py:87-110``)."""
    c = _cfg(config)
    return c.enabled and c.out_wgrad_fp8


def output_projection_dgrad(gradient: torch.Tensor, weight: torch.Tensor, return_quantized: bool = False,
                            config: Optional[Fp8BackwardConfig] = None):
    """``dy = gradient @ weight^T`` in FP8 (gradient [M, N_out], weight
    [K_in, N_out] as stored by the layer), or None to fall back to bf16.
    With ``return_quantized``: (dy, gradient_fp8, its decode scale), for a
    weight gradient that reuses the cast; the decode scale is then the one
    the payload was cast with even on a refresh call (the reference's
    out-wgrad path snapshots it the same way, ``ops/triton/bwd_fp8.py:1472-1482``)."""
    ops = output_projection_dgrad_operands(gradient, weight, snapshot_decode_scale=return_quantized, config=config)
    if ops is None:
        return None
    g8, gs, w8, ws = ops
    dy = fp8_dgrad(g8, gs, w8, ws, gradient.dtype if gradient.dtype == torch.bfloat16 else torch.bfloat16)
    return (dy, g8, gs) if return_quantized else dy


def output_projection_dgrad_operands(gradient: torch.Tensor, weight: torch.Tensor, snapshot_decode_scale: bool = True,
                                     config: Optional[Fp8BackwardConfig] = None):
    """The FP8 dgrad's operands (gradient e5m2 [M, N_out], its decode scale,
    weight^T e4m3 [K_in, N_out] as [N, K] rows, its scale), or None while the
    gradient's scale warms up (``output_projection_dgrad_operands``,
    ``ops/triton/bwd_fp8.py:1431``): the output projection dgrad runs on them, or
    the fused dgrad + LN * U * dropout backward does."""
    cfg = _cfg(config)
    if not cfg.enabled or not _has_stable_identity(weight):
        return None
    if gradient.dim() != 2 or gradient.shape[-1] % 128 or weight.shape[0] % 128:
        return None
    quantized = quantize_gradient("output_projection", gradient, discriminator=weight.data_ptr(),
                                  snapshot_decode_scale=snapshot_decode_scale, config=cfg)
    if quantized is None:
        return None
    g8, gs = quantized
    w8, ws = quantize_weight(weight)
    return g8, gs, w8, ws


def uvqk_fp8_backward_enabled(config: Optional[Fp8BackwardConfig] = None) -> bool:
    """The UVQK e5m2 dgrad arm (``DLRM_HSTU_FP8_BWD_UVQK=1`` with the e5m2 format)."""
    c = _cfg(config)
    return c.uvqk and c.grad_dtype == E5M2


def uvqk_wgrad_fp8t(config: Optional[Fp8BackwardConfig] = None) -> bool:
    """The UVQK weight gradient from the forward's e4m3 LN output and the e5m2
    gradient (``DLRM_HSTU_FP8_BWD_UVQK_WGRAD=fp8t``, ``uvqk_wgrad_fp8t``,
    ``ops/triton/bwd_fp8.py:1755-1762``)."""
    c = _cfg(config)
    return uvqk_fp8_backward_enabled(c) and c.uvqk_wgrad_fp8t


def uvqk_projection_backward(
    dz: Optional[torch.Tensor],
    normed_x: Optional[torch.Tensor],
    input_scale_value,
    weight: torch.Tensor,
    site: str = "uvqk_projection",
    per_layer: bool = True,
    normed_x_fp8_t: Optional[torch.Tensor] = None,
    recompute_normed_x: Optional[Callable[[], torch.Tensor]] = None,
    config: Optional[Fp8BackwardConfig] = None,
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
    ``uvqk_wgrad_fp8t``, ``normed_x_fp8_t`` (the forward's e4m3 LN output,
    here row-major [M, K] -- the kernel reads token rows directly, so no
    token-major copy is made) and ``input_scale_value`` (its dequantization
    scale: a float > 0 or a device fp32 tensor), the weight gradient is the
    FP8 product (x8 s_x)^T (dz8 s_dz) instead."""
    cfg = _cfg(config)
    if not uvqk_fp8_backward_enabled(cfg):
        return None
    if per_layer and not _has_stable_identity(weight):
        return None
    if (dz is None or dz.dim() != 2 or not dz.is_contiguous() or dz.dtype != torch.bfloat16 or dz.shape[1] % 256
            or dz.shape[0] == 0 or weight.dim() != 2 or weight.shape[1] != dz.shape[1] or weight.shape[0] % 128
            or (normed_x is None and recompute_normed_x is None)
            or (normed_x is not None and tuple(normed_x.shape) != (dz.shape[0], weight.shape[0]))):
        return None
    ctl = _registry.get(site, weight.data_ptr() if per_layer else None, dz.device)
    quantize, ends_window = ctl.admit(cfg)
    if not quantize:
        ctl.update(dz.detach().abs().amax(), cfg, roll=ends_window)
        return None
    dz8, amax, colsum = quantize_amax_colsum(dz, ctl.inv_scale, dtype=E5M2)
    # decode with the scale the payload was cast with (a refresh rewrites the live one)
    snap = ctl.update(amax, cfg, roll=ends_window, snapshot=ends_window)
    grad_scale = snap if snap is not None else ctl.scale
    w8, w_scale = quantize_weight(weight)
    sx = None
    if (uvqk_wgrad_fp8t(cfg) and normed_x_fp8_t is not None and normed_x_fp8_t.dtype == E4M3
            and tuple(normed_x_fp8_t.shape) == (dz.shape[0], weight.shape[0])):
        if torch.is_tensor(input_scale_value):
            sx = input_scale_value.reshape(-1)[:1].to(torch.float32)
        elif input_scale_value is not None and input_scale_value > 0.0:
            sx = torch.full((1,), float(input_scale_value), dtype=torch.float32, device=dz.device)
    if sx is not None:
        d_w = fp8_wgrad(normed_x_fp8_t, dz8, sx, grad_scale)
    else:
        xn = normed_x if normed_x is not None else recompute_normed_x()
        d_w = token_wgrad(xn, dz)
    d_x = fp8_dgrad(dz8, grad_scale, w8, w_scale)
    return d_x, d_w, colsum
