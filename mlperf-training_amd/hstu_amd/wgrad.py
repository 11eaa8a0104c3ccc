"""Weight gradients over the token axis, ``a^T b`` for row-major [T, N1] and
[T, N2] operands (one token per row), on this build's split-K kernel
(``hstu_wgrad``).

Reference call sites (paths relative to
``recommendation_v4/hstu/generative_recommenders/``):

* ``dw = torch.mm(x.t(), dz)`` of ``triton_addmm_bwd``
  (``ops/triton/triton_addmm.py:1737-1750``): the UVQK projection's wgrad;
* ``torch.mm(y.t(), dout)`` of the output block's backward
  (``ops/triton/triton_hstu_linear.py``): the output projection's wgrad;
* the split-K-over-tokens scheme with a fixed-order second pass of
  ``fp8_wgrad`` (``ops/triton/fp8_wgrad.py:27-160``).

* ``fp8_wgrad(a_fp8, b_fp8, scale_a, scale_b, out_dtype, split)``
  (``ops/triton/fp8_wgrad.py:109-160``): the same product from e4m3 A and
  e4m3 / e5m2 B, fp32 accumulation, both per-tensor scales applied at the
  end.  Row-major operands, as that kernel reads them (the token-major copies
  of its ``_tn`` variant are not needed).

``wgrad`` / ``fp8_wgrad`` raise when the library is missing; ``token_wgrad``
takes the kernel for the shapes it serves (N1, N2 multiples of 256, bf16)
and ``torch.mm`` on the device for any other.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib


_CODES = {torch.bfloat16: _lib.HSTU_DTYPE_BF16, torch.float8_e4m3fn: _lib.HSTU_DTYPE_FP8_E4M3,
          torch.float8_e5m2: _lib.HSTU_DTYPE_FP8_E5M2}


def supported(a: torch.Tensor, b: torch.Tensor) -> bool:
    """bf16 x bf16 or e4m3 x (e4m3 | e5m2) device operands [T, N1], [T, N2]
    with N1, N2 multiples of 256."""
    kinds = (a.dtype == torch.bfloat16 and b.dtype == torch.bfloat16) or (
        a.dtype == torch.float8_e4m3fn and b.dtype in (torch.float8_e4m3fn, torch.float8_e5m2))
    return (kinds and a.dim() == 2 and b.dim() == 2 and a.shape[0] == b.shape[0] and a.shape[1] % 256 == 0
            and b.shape[1] % 256 == 0 and a.is_cuda and b.is_cuda)


def _rows(t: torch.Tensor) -> torch.Tensor:
    ok = t.stride(1) == 1 and (t.stride(0) * t.element_size()) % 16 == 0 and t.data_ptr() % 16 == 0
    return t if ok else t.contiguous()


def wgrad(a: torch.Tensor, b: torch.Tensor, out_dtype: torch.dtype = torch.bfloat16, split: Optional[int] = None,
          scale_a: Optional[torch.Tensor] = None, scale_b: Optional[torch.Tensor] = None,
          with_colsum: bool = False):
    """``(a * scale_a)^T @ (b * scale_b)`` [N1, N2] with fp32 accumulation, for
    a [T, N1] and b [T, N2] both bf16, or e4m3 and e4m3 / e5m2; the scales are
    one-element fp32 device tensors or None (1).  ``split``: token ranges
    (None: about one workgroup per CU).  ``with_colsum`` (bf16): also the fp32
    column sums of b from the same pass, returned as (out, colsum)."""
    if not supported(a, b):
        raise NotImplementedError("hstu_wgrad takes bf16 x bf16 or e4m3 x e4m3/e5m2 [T, N1], [T, N2] device "
                                  "operands, N1, N2 % 256 == 0")
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise NotImplementedError("hstu_wgrad writes bf16 or fp32")
    a, b = _rows(a.detach()), _rows(b.detach())
    T, n1 = a.shape
    n2 = b.shape[1]
    sp = 0 if split is None else int(split)
    ws_bytes = int(_lib.fn("hstu_wgrad_workspace_bytes")(T, n1, n2, sp))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=a.device)
    out = torch.empty((n1, n2), dtype=out_dtype, device=a.device)
    sa = None if scale_a is None else scale_a.to(torch.float32).reshape(-1)[:1].contiguous()
    sb = None if scale_b is None else scale_b.to(torch.float32).reshape(-1)[:1].contiguous()
    code = _lib.HSTU_DTYPE_FP32 if out_dtype == torch.float32 else _lib.HSTU_DTYPE_BF16
    if with_colsum and b.dtype != torch.bfloat16:
        raise NotImplementedError("the fused column sum takes bf16 operands")
    colsum = torch.empty(n2, dtype=torch.float32, device=a.device) if with_colsum else None
    st = _lib.fn("hstu_wgrad")(
        _CODES[a.dtype], a.data_ptr(), a.stride(0), _CODES[b.dtype], b.data_ptr(), b.stride(0), T, n1, n2,
        None if sa is None else sa.data_ptr(), None if sb is None else sb.data_ptr(), out.data_ptr(), out.stride(0),
        code, None if colsum is None else colsum.data_ptr(), sp, ws.data_ptr(), ws_bytes,
        torch.cuda.current_stream(a.device).cuda_stream)
    _lib.check(st, "hstu_wgrad")
    return (out, colsum) if with_colsum else out


def fp8_wgrad(a_fp8: torch.Tensor, b_fp8: torch.Tensor, scale_a: torch.Tensor, scale_b: torch.Tensor,
              out_dtype: torch.dtype = torch.bfloat16, split: Optional[int] = None) -> torch.Tensor:
    """``(a_fp8 * scale_a)^T @ (b_fp8 * scale_b)`` [N1, N2]: e4m3 a [T, N1],
    e4m3 or e5m2 b [T, N2], one-element fp32 device scales (the reference's
    ``fp8_wgrad``).  Never syncs the host."""
    if a_fp8.dtype != torch.float8_e4m3fn or b_fp8.dtype not in (torch.float8_e4m3fn, torch.float8_e5m2):
        raise NotImplementedError("fp8_wgrad takes an e4m3 A and an e4m3 / e5m2 B")
    return wgrad(a_fp8, b_fp8, out_dtype=out_dtype, split=split, scale_a=scale_a, scale_b=scale_b)


def token_wgrad(a: torch.Tensor, b: torch.Tensor, with_colsum: bool = False):
    """``a^T b`` in bf16: the split-K kernel where it serves the shapes, else
    ``torch.mm``.  ``with_colsum``: (a^T b, fp32 column sums of b)."""
    if supported(a, b) and a.dtype == torch.bfloat16:
        return wgrad(a, b, with_colsum=with_colsum)
    out = torch.mm(a.t(), b)
    return (out, torch.sum(b, 0, dtype=torch.float32)) if with_colsum else out
