"""The C-ABI library without a GPU: it loads, exports every entry point
include/hstu_mi355x.h declares, and rejects bad arguments before any device
call (no compute is launched here)."""

import ctypes
import re
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
HEADER = REPO / "include" / "hstu_mi355x.h"


def _declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(hstu_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_expected_entry_points():
    names = _declared()
    for n in ("hstu_attn_fwd", "hstu_attn_fwd_workspace_bytes", "hstu_attn_bwd", "hstu_attn_bwd_dkdv", "hstu_attn_bwd_dq",
              "hstu_attn_bwd_workspace_bytes", "hstu_fp8_gemm_rowcol", "hstu_quantize_e4m3_rows", "hstu_version"):
        assert n in names


def test_library_exports_every_declared_symbol():
    import hstu_amd._lib as lib

    so = lib.load_library()
    for name in _declared():
        assert hasattr(so, name), name
    assert set(_declared()) == set(lib.EXPORTED_SYMBOLS)


def test_version_string():
    import hstu_amd._lib as lib

    v = lib.fn("hstu_version")()
    assert v.startswith(b"hstu-mi355x")


def test_workspace_size():
    import hstu_amd._lib as lib

    def a256(n):
        return (n + 255) // 256 * 256

    B, H = 10, 4
    cap = (B * H + 7) // 8
    sched = a256(4 * (8 * cap + 8 * (cap + 1) + 8 + 2 * B))  # items, starts, counts, per-sequence scratch
    f = lib.fn("hstu_attn_bwd_workspace_bytes")
    # dS tiles (8 KiB each) for the dQ kernel: 2 (ceil(N/128) + 1) (ceil(T/128) + B) per head, plus the
    # per-sequence tile prefix (int64 [B + 1])
    ds = a256((B + 1) * 8) + 2 * (4096 // 128 + 1) * ((1000 + 127) // 128 + B) * H * 8192
    dqb = a256((B + 1) * 8)  # the per-sequence dQ block prefix
    assert f(lib.HSTU_DTYPE_BF16, 1000, B, H, 128, 4096, 0) == sched + dqb + ds
    assert f(lib.HSTU_DTYPE_FP8_E4M3, 1000, B, H, 128, 4096, 0) == sched + 1000 * 4 * 128 * 2 + dqb + ds
    ext = a256(4 * (2 * 4096 + 256) * 4)  # pre-clamped bias rows, 2N+256 per head
    # bias-gradient rows (one per 128-query dQ block and head, 2R - 1 floats), their 64 chunk sums
    part = a256(((1000 + 127) // 128 + B) * H * (2 * 1024 - 1) * 4) + a256(64 * H * (2 * 1024 - 1) * 4)
    dq_base = a256((B + 1) * 8)
    assert f(lib.HSTU_DTYPE_BF16, 1000, B, H, 128, 4096, 1024) == sched + ext + part + dq_base + ds
    assert f(lib.HSTU_DTYPE_BF16, -1, B, H, 128, 4096, 0) == -1
    g = lib.fn("hstu_attn_fwd_workspace_bytes")
    assert g(lib.HSTU_DTYPE_BF16, 1000, B, H, 128, 4096) == sched
    assert g(lib.HSTU_DTYPE_FP8_E4M3, 1000, B, H, 128, 4096) == sched
    assert g(lib.HSTU_DTYPE_BF16, 1000, -1, H, 128, 4096) == -1


def test_bad_arguments_rejected_before_launch():
    import hstu_amd._lib as lib

    fwd = lib.fn("hstu_attn_fwd")
    # unknown dtype
    assert fwd(7, 16, 16, 16, 512, 512, 512, None, None, None, 0, 0, 16, 1, 4, 128, 64, 0.1,
               None, 0, 0, None, 0, 16, 512, 16, 4096, 1000, None) == lib.HSTU_E_BAD_ARG
    # row stride smaller than H*D
    assert fwd(0, 16, 16, 16, 100, 512, 512, None, None, None, 0, 0, 16, 1, 4, 128, 64, 0.1,
               None, 0, 0, None, 0, 16, 512, 16, 4096, 1000, None) == lib.HSTU_E_BAD_ARG
    # e4m3 without scales
    assert fwd(1, 16, 16, 16, 512, 512, 512, None, None, None, 0, 0, 16, 1, 4, 128, 64, 0.1,
               None, 0, 0, None, 0, 16, 512, 16, 4096, 1000, None) == lib.HSTU_E_BAD_ARG
    # unsupported head dim
    assert fwd(0, 16, 16, 16, 384, 384, 384, None, None, None, 0, 0, 16, 1, 4, 96, 64, 0.1,
               None, 0, 0, None, 0, 16, 384, 16, 4096, 1000, None) == lib.HSTU_E_UNSUPPORTED
    gemm = lib.fn("hstu_fp8_gemm_rowcol")
    # N not a multiple of 128
    assert gemm(16, 512, 16, 512, 16, 0, 16, 0, None, None, 0, 16, 100, 0, None, 8, 100, 512, 0, 0,
                None) == lib.HSTU_E_BAD_ARG
    q = lib.fn("hstu_quantize_e4m3_rows")
    assert q(16, 100, 4, 100, 7, None, 16, 100, 16, None) == lib.HSTU_E_BAD_ARG  # group not a multiple of 8


def test_missing_library_raises(tmp_path):
    import hstu_amd._lib as lib

    with pytest.raises(lib.HstuUnavailableError):
        lib.load_library.__wrapped__(tmp_path / "nope.so") if hasattr(lib.load_library, "__wrapped__") else \
            _load_fresh(lib, tmp_path / "nope.so")


def _load_fresh(lib, path):
    saved = lib._lib
    lib._lib = None
    try:
        return lib.load_library(path)
    finally:
        lib._lib = saved


def test_ln_mul_entry_points_reject_before_launch():
    import hstu_amd._lib as lib

    ws = lib.fn("hstu_ln_mul_bwd_workspace_bytes")
    assert ws(162251, 512) == 1024 * 2 * 512 * 4
    assert ws(10, 384) == -1 and ws(-1, 512) == -1
    fwd = lib.fn("hstu_ln_mul_fwd")
    X, W = 4096, 8192  # fake device addresses: none of these calls may launch

    def f(**kw):
        a = dict(x=X, ldx=512, u=X, ldu=512, w=W, b=W, pdt=lib.HSTU_DTYPE_BF16, eps=1e-6, rows=64, D=512, act=1,
                 silu_u=1, cu=1, cx=1,
                 training=0, ratio=0.0, seed=0, mask16=0, mask=None, ldm=0, y=X, ldy=1536, odt=0, inv=1.0,
                 out_scale=None, mean=W, rstd=W, stream=None)
        a.update(kw)
        return fwd(*a.values())

    assert f(D=384, ldx=384, ldu=384, ldy=3 * 384) == lib.HSTU_E_UNSUPPORTED
    assert f(ldy=1024) == lib.HSTU_E_BAD_ARG  # three 512-wide blocks do not fit
    assert f(act=3) == lib.HSTU_E_BAD_ARG
    assert f(odt=5) == lib.HSTU_E_BAD_ARG
    assert f(training=1, ratio=0.3) == lib.HSTU_E_BAD_ARG  # dropout without a mask buffer
    assert f(training=1, ratio=1.5, mask=X, ldm=512) == lib.HSTU_E_BAD_ARG
    assert f(x=X + 2) == lib.HSTU_E_UNSUPPORTED  # rows not 16-byte aligned
    assert f(rows=-1) == lib.HSTU_E_BAD_ARG
    assert f(pdt=lib.HSTU_DTYPE_FP8_E4M3) == lib.HSTU_E_BAD_ARG  # LayerNorm parameters are fp32 or bf16
    assert f(w=W + 8) == lib.HSTU_E_UNSUPPORTED  # parameters are read as 16-byte vectors
    mask = lib.fn("hstu_dropout_mask")
    assert mask(64, 512, 4, 0, 0.3, 1, X, 512, None) == lib.HSTU_E_BAD_ARG
    assert mask(64, 320, 1, 0, 0.3, 1, X, 320, None) == lib.HSTU_E_UNSUPPORTED
    bwd = lib.fn("hstu_ln_mul_bwd")

    def g(**kw):
        a = dict(dy=X, lddy=1536, x=X, ldx=512, u=X, ldu=512, w=W, b=W, pdt=lib.HSTU_DTYPE_FP32, mean=W, rstd=W,
                 rows=64, D=512, act=1,
                 silu_u=1, cu=1, cx=1, ratio=0.0, mask=None, ldm=0, dx=X, lddx=512, du=X, lddu=512, y=None, ldy=0,
                 dres=None, lddres=0, dw=W, db=W, ws=W, wsb=ws(64, 512), stream=None)
        a.update(kw)
        return bwd(*a.values())

    assert g(wsb=100) == lib.HSTU_E_BAD_ARG
    assert g(du=None) == lib.HSTU_E_BAD_ARG
    assert g(lddy=1024) == lib.HSTU_E_BAD_ARG
    assert g(y=X, ldy=512) == lib.HSTU_E_BAD_ARG
    assert g(D=128, ldx=128, ldu=128, lddx=128, lddu=128, lddy=384) == lib.HSTU_E_UNSUPPORTED
    assert g(dres=X, lddres=512) == lib.HSTU_E_BAD_ARG  # a residual gradient only without an x block
    assert g(cx=0, lddy=1024, dres=X, lddres=256) == lib.HSTU_E_BAD_ARG
    assert g(pdt=7) == lib.HSTU_E_BAD_ARG


def test_delta_entry_points_reject_before_launch():
    import hstu_amd._lib as lib

    wsq = lib.fn("hstu_delta_attn_workspace_bytes")
    assert wsq(128, 4, 128, 4096, 1) == 128 * 4 * 16 * 128 * 4
    assert wsq(-1, 4, 128, 4096, 1) == -1
    fwd = lib.fn("hstu_delta_attn_fwd")
    X, W = 4096, 8192

    def f(**kw):
        a = dict(dt=1, qdt=1, q=X, k=X, v=X, qrs=512, krs=512, vrs=512, qs=1.0, ks=1.0, vs=1.0, offs=W, B=8, H=4,
                 D=128, N=1024, ds=1, alpha=0.1, nt=None, win=0, ctx=0, out=X, ors=512, ws=W, wsb=wsq(8, 4, 128, 1024, 1),
                 stream=None)
        a.update(kw)
        return fwd(*a.values())

    assert f(D=96, qrs=384, krs=384, vrs=384, ors=384) == lib.HSTU_E_UNSUPPORTED
    assert f(wsb=16) == lib.HSTU_E_BAD_ARG
    assert f(dt=3) == lib.HSTU_E_BAD_ARG
    assert f(krs=100) == lib.HSTU_E_BAD_ARG
    assert f(k=X + 4) == lib.HSTU_E_UNSUPPORTED  # 8-element pieces must be aligned
    bwd = lib.fn("hstu_delta_attn_bwd")
    args = [1, 1, X, 512, X, X, X, 512, 512, 512, 1.0, 1.0, 1.0, W, 8, 4, 128, 1024, 5, 0.1, None, 0, 0, X, X, X,
            512, 512, 512, W, wsq(8, 4, 128, 1024, 5), None]
    assert bwd(*args) == lib.HSTU_E_UNSUPPORTED  # more than 4 delta rows per sequence


def test_do_quantizer_rejects_before_launch():
    import hstu_amd._lib as lib

    q = lib.fn("hstu_quantize_do_e4m3_blk")
    X, W = 4096, 8192

    def f(**kw):
        a = dict(dt=0, x=X, rs=512, offs=W, B=8, H=4, D=128, N=1024, y=X, e8=W, stream=None)
        a.update(kw)
        return q(*a.values())

    assert f(dt=1) == lib.HSTU_E_BAD_ARG          # e4m3 input
    assert f(rs=100) == lib.HSTU_E_BAD_ARG         # row stride below H * D
    assert f(N=0) == lib.HSTU_E_BAD_ARG
    assert f(D=96, rs=384) == lib.HSTU_E_UNSUPPORTED
    assert f(H=8, rs=1024) == lib.HSTU_E_UNSUPPORTED  # H * D = 1024
    assert f(x=X + 8) == lib.HSTU_E_UNSUPPORTED    # rows read as 16-byte pieces
    assert f(B=0) == 0


def test_colsum_cast_rejects_before_launch():
    import hstu_amd._lib as lib

    wsb = lib.fn("hstu_cast_fp8_amax_colsum_workspace_bytes")
    assert wsb(1000, 2048) == 2 * 2048 * 4 + 256          # 2 stripes of 512 rows; 16 amax partials -> 256 B
    assert wsb(0, 256) == 0
    assert wsb(10, 300) == -1 and wsb(-1, 256) == -1
    cast = lib.fn("hstu_cast_fp8_amax_colsum")
    X, W = 4096, 8192

    def f(**kw):
        a = dict(x=X, ldx=2048, rows=1000, cols=2048, inv=W, odt=lib.HSTU_DTYPE_FP8_E5M2, lim=57344.0, out=X,
                 rows_out=1000, colsum=W, amax=W, ws=W, wsb=wsb(1000, 2048), stream=None)
        a.update(kw)
        return cast(*a.values())

    assert f(odt=lib.HSTU_DTYPE_BF16) == lib.HSTU_E_BAD_ARG
    assert f(rows_out=999) == lib.HSTU_E_BAD_ARG             # padding rows below the input rows
    assert f(ldx=1024) == lib.HSTU_E_BAD_ARG
    assert f(lim=0.0) == lib.HSTU_E_BAD_ARG
    assert f(wsb=100) == lib.HSTU_E_BAD_ARG
    assert f(colsum=None) == lib.HSTU_E_BAD_ARG
    assert f(cols=300, ldx=304) == lib.HSTU_E_UNSUPPORTED    # columns in blocks of 256
    assert f(x=X + 8) == lib.HSTU_E_UNSUPPORTED              # 16-byte row pieces
    assert f(ldx=2052) == lib.HSTU_E_UNSUPPORTED


def test_wgrad_rejects_before_launch():
    import hstu_amd._lib as lib

    split = lib.fn("hstu_wgrad_split")
    wsb = lib.fn("hstu_wgrad_workspace_bytes")
    assert split(162251, 512, 2048, 0) == 16                 # 16 tiles -> one workgroup per CU
    assert split(1000, 512, 2048, 0) == 8                    # at least 4 k-steps of 32 tokens per split
    assert split(1000, 512, 2048, 1) == 1 and wsb(1000, 512, 2048, 1) == 0
    assert wsb(162251, 512, 2048, 0) == 16 * (512 + 1) * 2048 * 4       # product and column-sum partials
    assert split(100, 300, 256, 0) == -1 and split(0, 256, 256, 0) == 0
    f = lib.fn("hstu_wgrad")
    X, W = 4096, 8192
    bf, f32 = lib.HSTU_DTYPE_BF16, lib.HSTU_DTYPE_FP32

    def g(**kw):
        a = dict(adt=bf, A=X, lda=512, bdt=bf, B=X, ldb=2048, T=1000, N1=512, N2=2048, sa=None, sb=None, out=W,
                 ldo=2048, odt=bf, cs=None, split=0, ws=W, wsb=wsb(1000, 512, 2048, 0), stream=None)
        a.update(kw)
        return f(*a.values())

    assert g(odt=lib.HSTU_DTYPE_FP8_E4M3) == lib.HSTU_E_BAD_ARG
    assert g(lda=256) == lib.HSTU_E_BAD_ARG
    assert g(ldo=1024) == lib.HSTU_E_BAD_ARG
    assert g(T=-1) == lib.HSTU_E_BAD_ARG
    assert g(wsb=100) == lib.HSTU_E_BAD_ARG
    assert g(adt=lib.HSTU_DTYPE_FP8_E4M3) == lib.HSTU_E_UNSUPPORTED          # e4m3 x bf16
    e4, e5 = lib.HSTU_DTYPE_FP8_E4M3, lib.HSTU_DTYPE_FP8_E5M2
    assert g(adt=e5, bdt=e5) == lib.HSTU_E_UNSUPPORTED                     # A is e4m3 (the activation)
    assert g(adt=e4, bdt=e5, lda=520, ldb=2048) == lib.HSTU_E_UNSUPPORTED   # fp8 rows in 16-byte pieces
    assert g(N1=384, lda=384) == lib.HSTU_E_UNSUPPORTED       # 256-wide tiles
    assert g(A=X + 2) == lib.HSTU_E_UNSUPPORTED
    assert g(odt=f32, out=W + 8) == lib.HSTU_E_UNSUPPORTED    # fp32 rows stored 16 bytes at a time
    assert g(adt=e4, bdt=e5, cs=W) == lib.HSTU_E_UNSUPPORTED     # the fused column sum is bf16 only
    assert g(cs=W + 4) == lib.HSTU_E_UNSUPPORTED               # column sums stored 16 bytes at a time


def test_do_dequantizer_rejects_before_launch():
    import hstu_amd._lib as lib

    dq = lib.fn("hstu_dequantize_do_e4m3_blk")
    X, W = 4096, 8192
    assert dq(X, W, 10, 4, 128, X, 100, None) == lib.HSTU_E_BAD_ARG      # row stride below H * D
    assert dq(X, W, -1, 4, 128, X, 512, None) == lib.HSTU_E_BAD_ARG
    assert dq(X, W, 10, 4, 100, X, 400, None) == lib.HSTU_E_UNSUPPORTED  # D % 8
    assert dq(X + 4, W, 10, 4, 128, X, 512, None) == lib.HSTU_E_UNSUPPORTED
    assert dq(X, W, 0, 4, 128, X, 512, None) == 0


def test_noalloc_forward_rejects_before_launch():
    """The allocation-free forward refuses a call whose schedule would not
    fit its static scratch, and bad arguments, before touching a device."""
    import hstu_amd._lib as lib

    f = lib.fn("hstu_attn_fwd_noalloc")
    X = 4096  # fake device addresses: none of these calls may launch

    def call(B, H, D=128, dtype=lib.HSTU_DTYPE_BF16, rs=None, T=1000):
        rs = H * D if rs is None else rs
        return f(dtype, X, X, X, rs, rs, rs, None, None, None, 0, 0, X, B, H, D, 4096, 0.1, None, 0, 0, None, 0,
                 X, H * D, T, None)

    limit = 256 * 1024
    ws = lib.fn("hstu_attn_fwd_workspace_bytes")
    assert ws(0, 1000, 8192, 4, 128, 4096) > limit and ws(0, 1000, 6000, 4, 128, 4096) <= limit
    assert call(8192, 4) == lib.HSTU_E_SCRATCH_TOO_SMALL
    assert call(100, 4, D=96) == lib.HSTU_E_UNSUPPORTED
    assert call(100, 4, rs=100) == lib.HSTU_E_BAD_ARG                 # row stride < H * D
    assert call(100, 4, dtype=lib.HSTU_DTYPE_FP8_E4M3) == lib.HSTU_E_BAD_ARG  # e4m3 without scales
    assert call(100, 4, T=-1) == lib.HSTU_E_BAD_ARG
    assert call(0, 4) == 0                                            # empty batch: nothing to do


def test_outproj_ln_bwd_rejects_before_launch():
    """The fused output-projection backward's argument checks, on the CPU:
    every call below returns before any HIP call."""
    import hstu_amd._lib as lib

    ws = lib.fn("hstu_outproj_ln_bwd_workspace_bytes")
    assert ws(162251) == 256 * 2 * 512 * 4 and ws(-1) == -1
    f = lib.fn("hstu_outproj_ln_bwd")
    X, W = 4096, 8192  # fake device addresses: none of these calls may launch

    def g(**kw):
        a = dict(g8=X, ldg=512, gs=W, w8=X, ldw=512, ws_=W, x=X, ldx=512, u=X, ldu=512, w=W, b=W,
                 pdt=lib.HSTU_DTYPE_BF16, mean=W, rstd=W,
                 rows=64, D=512, act=1, silu_u=1, ratio=0.3, mask=X, ldm=512, dx=X, lddx=512, du=X, lddu=2048,
                 dw=W, db=W, ws=W, wsb=ws(64), stream=None)
        a.update(kw)
        return f(*a.values())

    assert g(wsb=100) == lib.HSTU_E_BAD_ARG
    assert g(u=None) == lib.HSTU_E_BAD_ARG  # the [u' | x | y] concat needs u
    assert g(gs=None) == lib.HSTU_E_BAD_ARG
    assert g(ldg=256) == lib.HSTU_E_BAD_ARG  # a gradient row is 512 bytes
    assert g(act=3) == lib.HSTU_E_BAD_ARG
    assert g(ratio=1.5) == lib.HSTU_E_BAD_ARG
    assert g(rows=-1) == lib.HSTU_E_BAD_ARG
    assert g(D=256, ldx=256, ldu=256, lddx=256, lddu=256, ldm=256) == lib.HSTU_E_UNSUPPORTED
    assert g(x=X + 2) == lib.HSTU_E_UNSUPPORTED  # rows not 16-byte aligned
    assert g(ldg=520) == lib.HSTU_E_UNSUPPORTED  # gradient rows not 16-byte aligned
    assert g(pdt=lib.HSTU_DTYPE_FP8_E5M2) == lib.HSTU_E_BAD_ARG


def test_fp8_pv_forward_declines_long_sequences_before_launch():
    """The FP8 P.V forward keeps a per-key table in LDS: past the N it can
    hold (hstu_attn_fwd_fp8_pv_max_seq_len) it returns HSTU_E_UNSUPPORTED
    before any device call, and the host's reason names it, so the op takes
    the bf16-P forward instead of failing."""
    import torch

    import hstu_amd._lib as lib
    from hstu_amd.hstu_attention import fp8_pv_fwd_reason

    n_max = lib.fn("hstu_attn_fwd_fp8_pv_max_seq_len")()
    assert 8192 <= n_max < 32768 and n_max % 64 == 0
    f = lib.fn("hstu_attn_fwd_fp8_pv")
    X = 4096  # fake device addresses: none of these calls may launch

    def call(N, B=10):
        return f(X, X, X, 512, 512, 512, X, X, X, 0, 0, X, B, 4, 128, N, 0.1, None, 0, 0, None, 0, 10.04,
                 X, 512, None, 0, 1000, None)

    assert call(n_max + 1) == lib.HSTU_E_UNSUPPORTED
    assert call(n_max + 1, B=0) == lib.HSTU_E_UNSUPPORTED
    assert call(n_max, B=0) == 0
    q = torch.zeros(4, 4, 128, dtype=torch.float8_e4m3fn)
    assert "LDS" in fp8_pv_fwd_reason(q, None, 0, 0, n_max + 64)
    assert fp8_pv_fwd_reason(q, None, 0, 0, n_max) is None
