"""Pins of the output-block oracle (oracle/hstu_ln_oracle.py), independent of
its own formulas: Random123 known-answer vectors for Philox4x32-10, Triton's
fp32 keep test for the integer threshold, the reference's compact-row mask
kernels as a second statement of the row layout, torch's layer_norm and
autograd / gradcheck, and closed forms."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import hstu_ln_oracle as L

# kat_vectors of the Random123 distribution, philox4x32 with 10 rounds:
# counter (4 words), key (2 words) -> output (4 words)
PHILOX_KAT = [
    ((0x00000000, 0x00000000, 0x00000000, 0x00000000), (0x00000000, 0x00000000),
     (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF), (0xFFFFFFFF, 0xFFFFFFFF),
     (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,expect", PHILOX_KAT)
def test_philox_known_answers(ctr, key, expect):
    out = L.philox4x32([np.array([c], dtype=np.uint64) for c in ctr], *key)
    assert tuple(int(w[0]) for w in out) == expect


def test_randint4x_uses_seed_words_as_key():
    # the seed's low word is k0, the high word k1 (triton_hstu_linear.py:296-300)
    seed = (0x299F31D0 << 32) | 0xA4093822
    off = np.array([0x243F6A88], dtype=np.int64)
    a = L.randint4x(seed, off)
    b = L.philox4x32((np.array([0x243F6A88]), np.zeros(1), np.zeros(1), np.zeros(1)), 0xA4093822, 0x299F31D0)
    assert all(int(x[0]) == int(y[0]) for x, y in zip(a, b))


@pytest.mark.parametrize("p", [0.0, 0.1, 0.3, 0.5, 0.7, 1e-9, 0.999999, 1.0])
def test_keep_above_matches_fp32_uniform_test(p):
    ka = L.mask_keep_above(p)
    rng = np.random.default_rng(0)
    xs = np.concatenate([rng.integers(0, 2 ** 31, 200000), np.arange(max(0, ka - 300), min(2 ** 31, ka + 300))])
    assert np.array_equal(xs > ka, L.uniform_keep(xs, p))
    if 0 <= ka < 2 ** 31 - 1:
        assert not L.uniform_keep(np.array([ka]), p)[0] and L.uniform_keep(np.array([ka + 1]), p)[0]


def test_keep_min16_closed_form():
    assert L.mask_keep_min16(0.0) == 0 and L.mask_keep_min16(1.0) == 65536
    assert L.mask_keep_min16(0.1) == 6554  # 0.1000061 (triton_hstu_linear.py:438-440)
    assert L.mask_keep_min16(0.3) == 19661


@pytest.mark.parametrize("mask16", [False, True])
@pytest.mark.parametrize("num_masks", [1, 2, 3])
def test_mask_rows_match_compact_row_restatement(mask16, num_masks):
    N, D, p, seed = 37, 256, 0.3, (7 << 40) + 12345
    full = L.dropout_mask(N, D, num_masks, p, seed, mask16)
    rows = [0, 3, 4, 7, 8, 13, 30, 36]
    assert np.array_equal(full[rows], L.dropout_mask_rows(rows, D, num_masks, p, seed, mask16))


@pytest.mark.parametrize("mask16", [False, True])
def test_mask_rates_and_extremes(mask16):
    N, D, nm, seed = 512, 512, 3, 2024
    m = L.dropout_mask(N, D, nm, 0.3, seed, mask16).astype(np.int64)
    n = N * D
    for j in range(nm):
        kept = ((m >> j) & 1).sum()
        assert abs(kept / n - 0.7) < 5 * np.sqrt(0.21 / n), (j, kept / n)
    # independent bits: P(both kept) ~ 0.49
    both = (((m >> 0) & (m >> 1) & 1).sum()) / n
    assert abs(both - 0.49) < 5 * np.sqrt(0.25 / n)
    assert (L.dropout_mask(16, 256, 3, 0.0, seed, mask16) == 7).all()
    assert (L.dropout_mask(16, 256, 3, 1.0, seed, mask16) == 0).all()
    # prefix property: a row's bits depend on its index only
    assert np.array_equal(L.dropout_mask(13, 256, 2, 0.3, seed, mask16),
                          L.dropout_mask(40, 256, 2, 0.3, seed, mask16)[:13])


def test_mask_seed_and_offsets_change_bits():
    a = L.dropout_mask(8, 256, 1, 0.5, 1, True)
    b = L.dropout_mask(8, 256, 1, 0.5, 2, True)
    c = L.dropout_mask(8, 256, 1, 0.5, 1 + (1 << 32), True)
    assert (a != b).mean() > 0.3 and (a != c).mean() > 0.3


def _inputs(N=24, D=256, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(N, D, generator=g, dtype=torch.float64) * 1.5 + 0.3
    u = torch.randn(N, D, generator=g, dtype=torch.float64)
    w = 1.0 + 0.2 * torch.randn(D, generator=g, dtype=torch.float64)
    b = 0.1 * torch.randn(D, generator=g, dtype=torch.float64)
    return x, u, w, b


def test_fwd_stats_and_plain_layernorm():
    x, u, w, b = _inputs()
    y, mean, rstd = L.ln_mul_dropout_fwd(x, None, w, b, 1e-6)
    xn = x.numpy()
    assert np.allclose(mean.numpy(), xn.mean(1), rtol=1e-13)
    assert np.allclose(rstd.numpy(), 1 / np.sqrt(xn.var(1) + 1e-6), rtol=1e-13)
    assert torch.allclose(y, F.layer_norm(x, (x.shape[1],), w, b, 1e-6))
    # u = 1 with no activation is plain LayerNorm; sigmoid(0) = 1/2
    y1, _, _ = L.ln_mul_dropout_fwd(x, torch.ones_like(u), w, b, 1e-6)
    assert torch.allclose(y1, y)
    y2, _, _ = L.ln_mul_dropout_fwd(x, torch.zeros_like(u), w, b, 1e-6, mul_u_activation_type="sigmoid")
    assert torch.allclose(y2, 0.5 * y)


@pytest.mark.parametrize("act", L.ACTS)
def test_fwd_concat_blocks(act):
    x, u, w, b = _inputs()
    D = x.shape[1]
    y, _, _ = L.ln_mul_dropout_fwd(x, u, w, b, 1e-6, silu_u=True, concat_u=True, concat_x=True,
                                   mul_u_activation_type=act)
    assert y.shape == (x.shape[0], 3 * D)
    assert torch.allclose(y[:, :D], u * torch.sigmoid(u), rtol=1e-14, atol=0) and torch.equal(y[:, D:2 * D], x)
    m = {"none": u, "silu": u * torch.sigmoid(u), "sigmoid": torch.sigmoid(u)}[act]
    ln = (x - x.mean(1, keepdim=True)) / torch.sqrt(x.var(1, unbiased=False, keepdim=True) + 1e-6) * w + b
    assert torch.allclose(y[:, 2 * D:], ln * m)
    yx, _, _ = L.ln_mul_dropout_fwd(x, u, w, b, 1e-6, concat_x=True)
    assert torch.equal(yx[:, :D], x)
    yu, _, _ = L.ln_mul_dropout_fwd(x, u, w, b, 1e-6, concat_u=True)
    assert torch.equal(yu[:, :D], u)


def test_fwd_dropout_closed_forms():
    x, u, w, b = _inputs()
    D = x.shape[1]
    kw = dict(silu_u=True, concat_u=True, concat_x=True, mul_u_activation_type="silu")
    y0, _, _ = L.ln_mul_dropout_fwd(x, u, w, b, 1e-6, **kw)
    keep = np.full(x.shape, 7, dtype=np.int8)
    y1, _, _ = L.ln_mul_dropout_fwd(x, u, w, b, 1e-6, dropout_ratio=0.3, mask=keep, **kw)
    assert torch.allclose(y1, y0 * float(L.dropout_scale(0.3)))
    y2, _, _ = L.ln_mul_dropout_fwd(x, u, w, b, 1e-6, dropout_ratio=0.3, mask=np.zeros(x.shape, np.int8), **kw)
    assert (y2 == 0).all()
    # bit 0 = y, bit 1 = x, bit 2 = u (triton_hstu_linear.py:630-650)
    only_x = np.full(x.shape, 2, dtype=np.int8)
    y3, _, _ = L.ln_mul_dropout_fwd(x, u, w, b, 1e-6, dropout_ratio=0.3, mask=only_x, **kw)
    assert (y3[:, :D] == 0).all() and (y3[:, 2 * D:] == 0).all()
    assert torch.allclose(y3[:, D:2 * D], x * float(L.dropout_scale(0.3)))


@pytest.mark.parametrize("act,silu_u,cu,cx", [("silu", True, True, True), ("none", False, True, True),
                                              ("sigmoid", False, False, True), ("none", False, True, False),
                                              ("silu", False, False, False)])
def test_bwd_gradcheck(act, silu_u, cu, cx):
    x, u, w, b = _inputs(N=6, D=16, seed=3)
    mask = L.dropout_mask(6, 16, 1 + cu + cx, 0.3, 99, True)
    kw = dict(dropout_ratio=0.3, mask=mask, silu_u=silu_u, concat_u=cu, concat_x=cx, mul_u_activation_type=act)

    def f(x_, u_, w_, b_):
        return L.ln_mul_dropout_fwd(x_, u_, w_, b_, 1e-5, **kw)[0]

    args = tuple(t.clone().requires_grad_(True) for t in (x, u, w, b))
    assert torch.autograd.gradcheck(f, args, eps=1e-6, atol=1e-6)
    dy = torch.randn(f(*args).shape, dtype=torch.float64)
    dx, du, dw, db = L.ln_mul_dropout_bwd(dy, x, u, w, b, 1e-5, **kw)
    ref = torch.autograd.grad(f(*args), args, dy)
    for a_, r_ in zip((dx, du, dw, db), ref):
        assert torch.allclose(a_, r_)


def test_bwd_plain_layernorm_matches_autograd_of_library_layernorm():
    x, _, w, b = _inputs(N=5, D=32, seed=5)
    dy = torch.randn(5, 32, dtype=torch.float64)
    dx, du, dw, db = L.ln_mul_dropout_bwd(dy, x, None, w, b, 1e-6)
    assert du is None
    xs, ws, bs = (t.clone().requires_grad_(True) for t in (x, w, b))
    F.layer_norm(xs, (32,), ws, bs, 1e-6).backward(dy)
    assert torch.allclose(dx, xs.grad) and torch.allclose(dw, ws.grad) and torch.allclose(db, bs.grad)


def test_e4m3_bytes_saturate_and_round():
    v = torch.tensor([0.0, 1.0, 1.0625, 1.1875, 500.0, -1000.0], dtype=torch.float64)
    q = L.e4m3_bytes(v, 1.0).to(torch.float32)
    assert q.tolist() == [0.0, 1.0, 1.0, 1.25, 448.0, -448.0]


def test_layer_oracle_composition_gradcheck():
    """The layer composition is differentiable end to end (gradcheck on a
    tiny unquantized instance: E = 8, one head of width 4, no dropout)."""
    from oracle import hstu_layer_oracle as LO

    lengths = np.array([3, 2])
    E, H, Dq, Dv = 8, 1, 4, 4
    p = LO.make_layer_params(E, H, Dq, Dv, seed=1, dtype=torch.float64)
    x = torch.randn(5, E, dtype=torch.float64, generator=torch.Generator().manual_seed(2))
    names = list(p)

    def f(x_, *ps):
        return LO.hstu_layer_ref(x_, dict(zip(names, ps)), lengths, 3, num_heads=H, attn_dim=Dq, hidden_dim=Dv,
                                 quantize=False)

    args = (x.requires_grad_(True),) + tuple(p[k].clone().requires_grad_(True) for k in names)
    assert torch.autograd.gradcheck(f, args, eps=1e-6, atol=1e-5)
    # the residual: d out / d x contains the identity
    out = f(*args)
    assert out.shape == x.shape


def test_layer_oracle_fp8_dgrad_matmul_is_dgrad_of_quantized_operands():
    """The layer oracle's FP8-dgrad projection: d(a) equals the bwd oracle's
    dgrad of the e5m2 gradient and per-tensor e4m3 weight, d(w) = a^T g
    exactly, and the forward is a @ w."""
    from oracle import hstu_bwd_fp8_oracle as BO
    from oracle import hstu_layer_oracle as LO

    g = torch.Generator().manual_seed(6)
    a = torch.randn(33, 64, generator=g, dtype=torch.float64, requires_grad=True)
    w = torch.randn(64, 96, generator=g, dtype=torch.float64, requires_grad=True)
    dz = torch.randn(33, 96, generator=g, dtype=torch.float64)
    s = float(dz.abs().max()) * 8 / 57344
    out = LO.fp8_dgrad_matmul(a, w, s)
    assert torch.equal(out.detach(), (a @ w).detach())
    out.backward(dz)
    g8 = (dz / s).to(torch.float8_e5m2)
    ws = float(w.detach().abs().max().float() / 448)
    w8 = (w.detach() / ws).to(torch.float8_e4m3fn)
    assert torch.allclose(a.grad, BO.dgrad(g8, s, w8, ws), rtol=1e-12, atol=0)
    assert torch.allclose(w.grad, a.detach().t() @ dz, rtol=1e-12, atol=0)
    rel = float((a.grad - dz @ w.detach().t()).norm() / (dz @ w.detach().t()).norm())
    assert 1e-3 < rel < 0.1                                                    # quantized, but close
    assert LO.fp8_dgrad_matmul(a, w, None).grad_fn is not None



def test_layer_oracle_fp8_wgrad_matmul_is_wgrad_of_quantized_operands():
    """With an activation scale the oracle's weight gradient is the bwd
    oracle's wgrad of the e4m3 activation and the e5m2 gradient."""
    from oracle import hstu_bwd_fp8_oracle as BO
    from oracle import hstu_layer_oracle as LO

    g = torch.Generator().manual_seed(8)
    a = torch.randn(40, 64, generator=g, dtype=torch.float64, requires_grad=True)
    w = torch.randn(64, 32, generator=g, dtype=torch.float64, requires_grad=True)
    dz = torch.randn(40, 32, generator=g, dtype=torch.float64)
    s_g, s_a = float(dz.abs().max()) * 8 / 57344, float(a.detach().abs().max()) / 448
    LO.fp8_dgrad_matmul(a, w, s_g, s_a).backward(dz)
    a8 = (a.detach() / s_a).to(torch.float8_e4m3fn)
    g8 = (dz / s_g).to(torch.float8_e5m2)
    assert torch.allclose(w.grad, BO.wgrad(a8, g8, s_a, s_g), rtol=1e-12, atol=0)
    rel = float((w.grad - a.detach().t() @ dz).norm() / (a.detach().t() @ dz).norm())
    assert 1e-3 < rel < 0.1
