"""Pins of the CPU oracle (oracle/hstu_oracle.py), independent of its own
formulas: brute-force loops, closed forms, library routines (torch autograd /
gradcheck, torch's e4m3fn conversion) and the documented config generator
outputs.  Each check is chosen so that a plausible slip (dropped 1/N, alpha
applied twice, off-by-one in the mask diagonal, transposed operand) fails."""

import math

import numpy as np
import pytest
import torch

from oracle import hstu_oracle as orc


def _rand(lengths, H, D, seed=0, std=0.7):
    q, k, v = orc.make_qkv(lengths, H, D, std, seed=seed, dtype=torch.float64)
    return q, k, v, orc.offsets_from_lengths(lengths)


# ---------------------------------------------------------------- generators
def test_config_generators_match_baseline():
    L1 = orc.lengths_for_config(1)
    assert L1.tolist() == [221, 169, 139, 81, 90, 25, 34, 19] and L1.sum() == 778
    assert orc.lengths_for_config(2).sum() == 37429
    L3 = orc.lengths_for_config(3)
    assert L3.sum() == 162251 and len(L3) == 128
    assert orc.causal_pairs(L3) == 300720505
    # config 3 fwd+bwd FLOPs (2.156 TFLOP; fwd 0.616, bwd 1.540)
    assert abs(orc.attn_flops(L3, 4, 128) / 1e12 - 2.156) < 1e-3
    assert abs(orc.attn_flops(L3, 4, 128, bwd=False) / 1e12 - 0.616) < 1e-3


# ---------------------------------------------------------------- jagged <-> padded
def test_jagged_padded_roundtrip_and_truncation():
    lengths = [3, 0, 5, 2]
    offs = orc.offsets_from_lengths(lengths)
    x = torch.arange(10 * 3, dtype=torch.float64).reshape(10, 3)
    d = orc.jagged_to_padded(x, offs, 4)
    assert d.shape == (4, 4, 3)
    assert torch.equal(d[2, :4], x[3:7]) and torch.all(d[1] == 0) and torch.all(d[0, 3] == 0)
    back = orc.padded_to_jagged(d, offs, 10)
    assert torch.equal(back[:3], x[:3]) and torch.equal(back[3:7], x[3:7])
    assert torch.all(back[7] == 0)  # position 4 of sequence 2 is beyond N=4
    assert torch.equal(back[8:], x[8:])


# ---------------------------------------------------------------- mask
def test_mask_plain_causal_is_lower_triangle():
    N = 9
    m = orc.valid_attn_mask(N, torch.tensor([9]))
    assert torch.equal(m[0], torch.tril(torch.ones(N, N, dtype=torch.bool)))


def test_mask_one_target_equals_causal():
    N = 7
    lengths = torch.tensor([7, 5])
    a = orc.valid_attn_mask(N, lengths, num_targets=torch.tensor([1, 1]))
    b = orc.valid_attn_mask(N, lengths).expand(2, N, N)
    for s, L in enumerate(lengths.tolist()):  # positions >= L are padding
        assert torch.equal(a[s, :L, :L], b[s, :L, :L])


def test_mask_targets_closed_form():
    """Targets (last nt positions) see every non-target key before them and
    themselves, never another target."""
    N, L, nt = 10, 10, 3
    m = orc.valid_attn_mask(N, torch.tensor([L]), num_targets=torch.tensor([nt]))[0]
    for i in range(L):
        for j in range(L):
            if i < L - nt:
                want = j <= i
            else:
                want = (j < L - nt) or (j == i)
            assert bool(m[i, j]) == want, (i, j)


def test_mask_max_attn_len_band():
    N, M = 12, 3
    m = orc.valid_attn_mask(N, torch.tensor([N]), max_attn_len=M)[0]
    i, j = torch.meshgrid(torch.arange(N), torch.arange(N), indexing="ij")
    assert torch.equal(m, (j <= i) & (i - j <= M))


def test_mask_contextual_rows_see_all():
    """With contextual_seq_len c, rows 0..c-1 share id 0 and attend to every
    column of the sequence (the prefix is global context)."""
    N, c = 8, 3
    m = orc.valid_attn_mask(N, torch.tensor([N]), contextual_seq_len=c)[0]
    assert bool(m[:c].all())
    assert torch.equal(m[c:], torch.tril(torch.ones(N, N, dtype=torch.bool))[c:] | (torch.arange(N) < c))


def test_mask_scalar_matches_tensor_form():
    N = 11
    for nt, mal, ctx in [(None, 0, 0), (2, 0, 0), (None, 4, 0), (None, 0, 3), (3, 5, 2)]:
        L = 9
        m = orc.valid_attn_mask(N, torch.tensor([L]), None if nt is None else torch.tensor([nt]), mal, ctx)[0]
        for i in range(L):
            for j in range(L):
                assert bool(m[i, j]) == orc.valid_pair(i, j, L, nt, mal, ctx), (nt, mal, ctx, i, j)


# ---------------------------------------------------------------- forward
@pytest.mark.parametrize("kw", [{}, {"num_targets": [2, 1, 4]}, {"max_attn_len": 3},
                                {"contextual_seq_len": 2}, {"attn_bias": True}])
def test_dense_equals_bruteforce_loop(kw):
    lengths = [6, 1, 9]
    H, D, N = 2, 5, 11
    q, k, v, offs = _rand(lengths, H, D)
    bias = orc.make_bias(H, 4, seed=2, std=0.5).double() if kw.pop("attn_bias", False) else None
    nt = kw.pop("num_targets", None)
    nt_t = None if nt is None else torch.tensor(nt)
    a = orc.hstu_mha_dense(N, 0.3, q, k, v, offs, nt_t, attn_bias=bias, dtype=torch.float64, **kw)
    b = orc.hstu_mha_loop(N, 0.3, q.numpy(), k.numpy(), v.numpy(), offs.numpy(),
                          None if nt is None else np.array(nt), attn_bias=None if bias is None else bias.numpy(),
                          **kw)
    assert np.abs(a.numpy() - b).max() < 1e-12


def test_single_token_closed_form():
    q, k, v, offs = _rand([1], 1, 4)
    N, alpha = 7, 0.4
    x = alpha * float(q[0, 0] @ k[0, 0])
    want = x / (1 + math.exp(-x)) / N * v[0, 0]
    got = orc.hstu_mha_dense(N, alpha, q, k, v, offs, dtype=torch.float64)[0, 0]
    assert torch.allclose(got, want, atol=1e-14)


def test_alpha_zero_gives_zero_and_linearity_in_v():
    q, k, v, offs = _rand([5, 3], 2, 4)
    z = orc.hstu_mha_dense(5, 0.0, q, k, v, offs, dtype=torch.float64)
    assert torch.all(z == 0)  # silu(0) = 0
    a = orc.hstu_mha_dense(5, 0.5, q, k, v, offs, dtype=torch.float64)
    b = orc.hstu_mha_dense(5, 0.5, q, k, 2.0 * v + 1.0, offs, dtype=torch.float64)
    c = orc.hstu_mha_dense(5, 0.5, q, k, torch.ones_like(v), offs, dtype=torch.float64)
    assert torch.allclose(b, 2 * a + c, atol=1e-13)


def test_causal_prefix_invariance_and_n_scaling():
    q, k, v, offs = _rand([8], 1, 4)
    base = orc.hstu_mha_dense(8, 0.5, q, k, v, offs, dtype=torch.float64)
    k2, v2 = k.clone(), v.clone()
    k2[5:] += 3.0
    v2[5:] -= 2.0
    pert = orc.hstu_mha_dense(8, 0.5, q, k2, v2, offs, dtype=torch.float64)
    assert torch.equal(base[:5], pert[:5]) and not torch.allclose(base[5:], pert[5:])
    # N enters only as 1/N (as long as every length <= N)
    big = orc.hstu_mha_dense(16, 0.5, q, k, v, offs, dtype=torch.float64)
    assert torch.allclose(big * 16, base * 8, atol=1e-13)


def test_jagged_independence():
    lengths = [4, 6]
    q, k, v, offs = _rand(lengths, 2, 3)
    both = orc.hstu_mha_dense(6, 0.7, q, k, v, offs, dtype=torch.float64)
    one = orc.hstu_mha_dense(6, 0.7, q[4:], k[4:], v[4:], orc.offsets_from_lengths([6]), dtype=torch.float64)
    assert torch.allclose(both[4:], one, atol=1e-14)


# ---------------------------------------------------------------- backward
def test_backward_autograd_matches_closed_form():
    lengths = [5, 3, 7]
    q, k, v, offs = _rand(lengths, 2, 4)
    dout = torch.randn(q.shape, generator=torch.Generator().manual_seed(3), dtype=torch.float64)
    bias = orc.make_bias(2, 4, seed=9, std=0.5).double()
    a = orc.hstu_mha_bwd(7, 0.4, q, k, v, offs, dout, attn_bias=bias)
    b = orc.hstu_mha_bwd_closed_form(7, 0.4, q, k, v, offs, dout, attn_bias=bias)
    for x, y in zip(a, b):
        assert torch.allclose(x, y, atol=1e-12)


def test_backward_gradcheck():
    lengths = [3, 4]
    q, k, v, offs = _rand(lengths, 1, 3)
    bias = orc.make_bias(1, 3, seed=4, std=0.5).double()
    for t in (q, k, v, bias):
        t.requires_grad_(True)
    fn = lambda q_, k_, v_, b_: orc.hstu_mha_dense(4, 0.6, q_, k_, v_, offs, attn_bias=b_,  # noqa: E731
                                                    dtype=torch.float64)
    assert torch.autograd.gradcheck(fn, (q, k, v, bias), eps=1e-6, atol=1e-8)


# ---------------------------------------------------------------- bias
def test_bias_index_clamps_and_dense_bias_matches_loop():
    R, N, H = 3, 6, 2
    tab = torch.arange(H * (2 * R - 1), dtype=torch.float64).reshape(H, 2 * R - 1)
    db = orc.dense_bias(tab, N)
    for h in range(H):
        for i in range(N):
            for j in range(N):
                off = max(-(R - 1), min(R - 1, i - j))
                assert db[h, i, j] == tab[h, off + R - 1]


# ---------------------------------------------------------------- quantizers
def test_quantizer_closed_form_and_torch_conversion():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(6, 3, 16, generator=g) * 4
    x[0, 0] = 0
    q8, s = orc.quantize_e4m3_rows(x, dim=-1)
    amax = x.abs().amax(-1)
    assert torch.equal(s, torch.where(amax > 0, amax / 448.0, torch.full_like(amax, 1 / 448.0)))
    # the group maximum maps exactly onto 448 and survives the conversion
    nz = amax > 0
    assert torch.equal(q8.float().abs().amax(-1)[nz], torch.full_like(amax[nz], 448.0))
    # dequantization error is within half an e4m3 step (2^-4 relative) or the subnormal step
    dq = orc.dequantize(q8, s)
    err = (dq - x).abs()
    assert bool((err <= x.abs() * 2.0 ** -4 + s.unsqueeze(-1) * 2.0 ** -10).all())


def test_per_tensor_quantizer_margin():
    x = torch.randn(50, 8, generator=torch.Generator().manual_seed(6))
    q8, s = orc.quantize_e4m3_per_tensor(x, margin=1.5)
    assert torch.allclose(s, (x.abs().max() * 1.5 / 448).reshape(1, 1))
    assert float(q8.float().abs().max()) <= 448 / 1.5 + 16


# ---------------------------------------------------------------- FP8 GEMM
def test_rowcol_gemm_matches_matmul():
    g = torch.Generator().manual_seed(7)
    a = torch.randn(9, 32, generator=g)
    w = torch.randn(32, 16, generator=g)
    a8, sa = orc.quantize_e4m3_rows(a, dim=1)
    w8t, sw = orc.quantize_e4m3_rows(w.t().contiguous(), dim=1)
    bias = torch.randn(16, generator=g)
    res = torch.randn(9, 16, generator=g)
    c = orc.fp8_rowcol_gemm(a8, sa, w8t.t(), sw, bias=bias, silu_cols=(0, 4), residual=res)
    ad = a8.double() * sa.double().reshape(-1, 1)
    wd = (w8t.double() * sw.double().reshape(-1, 1)).t()
    want = ad @ wd + bias.double()
    want[:, :4] = torch.nn.functional.silu(want[:, :4])
    want = want + res.double()
    assert torch.allclose(c, want, atol=1e-12)
    # and the dequantized product approximates the unquantized one
    assert orc.rel_l2(a.double() @ w.double(), ad @ wd) < 0.06


# ---------------------------------------------------------------- delta-q attention
@pytest.mark.parametrize("ds,nt,ctx,win", [(1, None, 0, 0), (2, None, 0, 0), (1, [1, 2, 1], 0, 0), (3, None, 2, 3)])
def test_cached_attention_equals_last_rows_of_full(ds, nt, ctx, win):
    lengths = [9, 5, 12]
    H, D, N = 2, 8, 12
    q, k, v, offs = _rand(lengths, H, D, seed=4)
    num_targets = None if nt is None else torch.tensor(nt)
    full = orc.hstu_mha_dense(N, 0.3, q, k, v, offs, num_targets=num_targets, max_attn_len=win,
                              contextual_seq_len=ctx, dtype=torch.float64)
    rows = torch.cat([torch.arange(int(offs[b + 1]) - ds, int(offs[b + 1])) for b in range(len(lengths))])
    got = orc.cached_hstu_mha(N, 0.3, q[rows], k, v, offs, num_targets=num_targets, max_attn_len=win,
                              contextual_seq_len=ctx)
    assert torch.allclose(got, full[rows], rtol=1e-12, atol=1e-14)


def test_cached_attention_backward_matches_full_backward_on_delta_rows():
    lengths = [7, 11]
    H, D, N, ds = 2, 8, 11, 1
    q, k, v, offs = _rand(lengths, H, D, seed=6)
    rows = torch.cat([torch.arange(int(offs[b + 1]) - ds, int(offs[b + 1])) for b in range(len(lengths))])
    dout_d = torch.randn(len(rows), H, D, dtype=torch.float64, generator=torch.Generator().manual_seed(2))
    dout = torch.zeros_like(q)
    dout[rows] = dout_d
    rq, rk, rv, _ = orc.hstu_mha_bwd(N, 0.25, q, k, v, offs, dout, dtype=torch.float64)
    qd = q[rows].clone().requires_grad_(True)
    kk, vv = k.clone().requires_grad_(True), v.clone().requires_grad_(True)
    orc.cached_hstu_mha(N, 0.25, qd, kk, vv, offs).backward(dout_d)
    assert torch.allclose(qd.grad, rq[rows]) and torch.allclose(kk.grad, rk) and torch.allclose(vv.grad, rv)
