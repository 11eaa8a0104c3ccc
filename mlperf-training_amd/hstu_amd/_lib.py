"""Loader for the C-ABI library ``libhstu_mi355x.so`` (declared in
``include/hstu_mi355x.h``).

The library is built ahead of time (``mlperf-training_amd/build.py``) and
bound with ctypes, the same FFI the reference uses for its native kernels
(``ops/hip/k512_fp8_gemm.py:260-270``).  There is no fallback: if the library
is missing or does not load, every entry point raises ``HstuUnavailableError``
(mirroring ``FlyDSLUnavailableError``, ``ops/flydsl/hstu_flydsl_mha.py:183-188``).
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path
from typing import Optional

LIB_NAME = "libhstu_mi355x.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME

HSTU_DTYPE_BF16 = 0
HSTU_DTYPE_FP8_E4M3 = 1
HSTU_DTYPE_FP32 = 2
HSTU_DTYPE_FP8_E5M2 = 3
HSTU_E_BAD_ARG = -1
HSTU_E_UNSUPPORTED = -2
HSTU_E_SCRATCH_TOO_SMALL = -3

# Every extern "C" symbol include/hstu_mi355x.h declares.
EXPORTED_SYMBOLS = (
    "hstu_version",
    "hstu_attn_fwd",
    "hstu_attn_fwd_fp8_pv",
    "hstu_attn_fwd_fp8_pv_max_seq_len",
    "hstu_attn_bwd",
    "hstu_attn_fwd_workspace_bytes",
    "hstu_attn_bwd_workspace_bytes",
    "hstu_attn_bwd_dkdv",
    "hstu_attn_bwd_dq",
    "hstu_fp8_gemm_rowcol",
    "hstu_quantize_e4m3_rows",
    "hstu_dropout_mask",
    "hstu_ln_mul_fwd",
    "hstu_ln_mul_bwd_workspace_bytes",
    "hstu_ln_mul_bwd",
    "hstu_outproj_ln_bwd_workspace_bytes",
    "hstu_outproj_ln_bwd",
    "hstu_delta_attn_workspace_bytes",
    "hstu_delta_attn_fwd",
    "hstu_delta_attn_bwd",
    "hstu_quantize_do_e4m3_blk",
    "hstu_dequantize_do_e4m3_blk",
    "hstu_fp8_gemm",
    "hstu_bf16_gemm",
    "hstu_cast_fp8_amax_partials",
    "hstu_cast_fp8_amax",
    "hstu_quantize_e4m3_unit",
    "hstu_fp8_site_update",
    "hstu_cast_fp8_amax_colsum_workspace_bytes",
    "hstu_cast_fp8_amax_colsum",
    "hstu_wgrad_split",
    "hstu_wgrad_workspace_bytes",
    "hstu_wgrad",
    "hstu_attn_fwd_noalloc",
    "hstu_attn_bwd_fp8",
    "hstu_attn_bwd_fp8_workspace_bytes",
    "hstu_attn_bwd_fp8_dkdv",
    "hstu_attn_bwd_fp8_dq",
)


class HstuUnavailableError(RuntimeError):
    """The native library cannot run on this host (missing build, no GPU)."""


class HstuKernelError(RuntimeError):
    """A C-ABI entry point returned a non-zero status."""


_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_u64 = ctypes.c_uint64

_SIGNATURES = {
    "hstu_version": (ctypes.c_char_p, []),
    "hstu_attn_fwd_fp8_pv_max_seq_len": (ctypes.c_int32, []),
    "hstu_attn_fwd": (
        _i32,
        [_i32, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _i64, _vp, _i32, _i32, _i32, _i32,
         _f32, _vp, _i32, _i32, _vp, _i32, _vp, _i64, _vp, _i64, _i64, _vp],
    ),
    "hstu_attn_fwd_fp8_pv": (
        _i32,
        [_vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _i64, _vp, _i32, _i32, _i32, _i32,
         _f32, _vp, _i32, _i32, _vp, _i32, _f32, _vp, _i64, _vp, _i64, _i64, _vp],
    ),
    "hstu_attn_fwd_workspace_bytes": (_i64, [_i32, _i64, _i32, _i32, _i32, _i32]),
    "hstu_attn_fwd_noalloc": (
        _i32,
        [_i32, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _i64, _vp, _i32, _i32, _i32, _i32,
         _f32, _vp, _i32, _i32, _vp, _i32, _vp, _i64, _i64, _vp],
    ),
    "hstu_attn_bwd": (
        _i32,
        [_i32, _vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _i64, _vp, _i32, _i32, _i32,
         _i32, _f32, _vp, _i32, _i32, _vp, _i32, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _i64, _i64, _vp],
    ),
    "hstu_attn_bwd_workspace_bytes": (_i64, [_i32, _i64, _i32, _i32, _i32, _i32, _i32]),
    "hstu_attn_bwd_fp8_workspace_bytes": (_i64, [_i64, _i32, _i32, _i32, _i32, _i32]),
    "hstu_attn_bwd_fp8": (
        _i32,
        [_vp, _vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _i64, _vp, _i32, _i32, _i32, _i32,
         _f32, _i32, _i32, _vp, _i32, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _i64, _i64, _vp],
    ),
    "hstu_attn_bwd_fp8_dkdv": "hstu_attn_bwd_fp8",
    "hstu_attn_bwd_fp8_dq": "hstu_attn_bwd_fp8",
    "hstu_attn_bwd_dkdv": None,
    "hstu_attn_bwd_dq": None,
    "hstu_fp8_gemm_rowcol": (
        _i32,
        [_vp, _i64, _vp, _i64, _vp, _i32, _vp, _i32, _vp, _vp, _i64, _vp, _i64, _i32, _vp,
         _i32, _i32, _i32, _i32, _i32, _vp],
    ),
    "hstu_fp8_gemm": (
        _i32,
        [_i32, _vp, _i64, _vp, _i64, _vp, _i32, _vp, _i32, _vp, _vp, _i64, _vp, _i64, _i32, _vp,
         _i32, _i32, _i32, _i32, _i32, _vp],
    ),
    "hstu_bf16_gemm": (_i32, [_vp, _i64, _vp, _i64, _vp, _vp, _i64, _vp, _i64, _i32, _i32, _i32, _i32, _i32, _vp]),
    "hstu_cast_fp8_amax_partials": (_i64, [_i64]),
    "hstu_cast_fp8_amax": (_i32, [_i32, _vp, _i64, _vp, _i32, _f32, _vp, _vp, _i64, _vp]),
    "hstu_quantize_e4m3_unit": (_i32, [_i32, _vp, _i64, _vp, _vp, _vp, _i64, _vp]),
    "hstu_fp8_site_update": (_i32, [_vp, _i32, _vp, _f32, _i32, _i32, _f32, _vp, _vp]),
    "hstu_cast_fp8_amax_colsum_workspace_bytes": (_i64, [_i64, _i64]),
    "hstu_wgrad_split": (_i32, [_i64, _i32, _i32, _i32]),
    "hstu_wgrad_workspace_bytes": (_i64, [_i64, _i32, _i32, _i32]),
    "hstu_wgrad": (_i32, [_i32, _vp, _i64, _i32, _vp, _i64, _i64, _i32, _i32, _vp, _vp, _vp, _i64, _i32, _vp, _i32,
                          _vp, _i64, _vp]),
    "hstu_cast_fp8_amax_colsum": (_i32, [_vp, _i64, _i64, _i64, _vp, _i32, _f32, _vp, _i64, _vp, _vp, _vp, _i64,
                                         _vp]),
    "hstu_quantize_e4m3_rows": (
        _i32,
        [_vp, _i64, _i32, _i32, _i32, _vp, _vp, _i64, _vp, _vp],
    ),
    "hstu_dropout_mask": (_i32, [_i32, _i32, _i32, _i32, _f32, _u64, _vp, _i64, _vp]),
    "hstu_ln_mul_fwd": (
        _i32,
        [_vp, _i64, _vp, _i64, _vp, _vp, _i32, _f32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _u64, _i32,
         _vp, _i64, _vp, _i64, _i32, _f32, _vp, _vp, _vp, _vp],
    ),
    "hstu_ln_mul_bwd_workspace_bytes": (_i64, [_i32, _i32]),
    "hstu_delta_attn_workspace_bytes": (_i64, [_i32, _i32, _i32, _i32, _i32]),
    "hstu_delta_attn_fwd": (
        _i32,
        [_i32, _i32, _vp, _vp, _vp, _i64, _i64, _i64, _f32, _f32, _f32, _vp, _i32, _i32, _i32, _i32, _i32, _f32,
         _vp, _i32, _i32, _vp, _i64, _vp, _i64, _vp],
    ),
    "hstu_delta_attn_bwd": (
        _i32,
        [_i32, _i32, _vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _f32, _f32, _f32, _vp, _i32, _i32, _i32, _i32,
         _i32, _f32, _vp, _i32, _i32, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _i64, _vp],
    ),
    "hstu_quantize_do_e4m3_blk": (_i32, [_i32, _vp, _i64, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp]),
    "hstu_dequantize_do_e4m3_blk": (_i32, [_vp, _vp, _i64, _i32, _i32, _vp, _i64, _vp]),
    "hstu_ln_mul_bwd": (
        _i32,
        [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _i32, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _f32,
         _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _vp],
    ),
    "hstu_outproj_ln_bwd_workspace_bytes": (_i64, [_i32]),
    "hstu_outproj_ln_bwd": (
        _i32,
        [_vp, _i64, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _i64, _vp, _vp, _i32, _vp, _vp, _i32, _i32, _i32, _i32,
         _f32, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _vp],
    ),
}


def load_library(path: Optional[Path] = None) -> ctypes.CDLL:
    """Load (once per process) and return the bound library."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        p = Path(path) if path is not None else LIB_PATH
        if not p.exists():
            raise HstuUnavailableError(
                f"{p} is not built; run `python mlperf-training_amd/build.py` "
                "(or __graft_entry__.build()) first.  There is no fallback path."
            )
        try:
            lib = ctypes.CDLL(str(p))
        except OSError as e:  # pragma: no cover - depends on host
            raise HstuUnavailableError(f"cannot load {p}: {e}") from e
        _lib = lib
        return lib


_bound = {}


def fn(name: str):
    """The typed ctypes function for one exported symbol."""
    f = _bound.get(name)
    if f is None:
        f = getattr(load_library(), name)
        sig = _SIGNATURES[name] or _SIGNATURES["hstu_attn_bwd"]
        if isinstance(sig, str):  # same argument list as another entry point
            sig = _SIGNATURES[sig]
        res, args = sig
        f.restype = res
        f.argtypes = args
        _bound[name] = f
    return f


def check(status: int, what: str) -> None:
    if status != 0:
        msg = {HSTU_E_BAD_ARG: "bad argument", HSTU_E_UNSUPPORTED: "unsupported shape/layout",
               HSTU_E_SCRATCH_TOO_SMALL: "needs more than the allocation-free entry point's scratch"}.get(
            status, f"hipError {status}")
        raise HstuKernelError(f"{what} failed: {msg}")


def ptr(t) -> Optional[int]:
    """Device address of a tensor (None for None)."""
    return None if t is None else t.data_ptr()
