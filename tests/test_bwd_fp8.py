"""FP8 backward projection arm (e5m2 output-projection dgrad): the oracle and
the delayed-scale controller on the CPU, the one-pass cast (bit-exact), the
e5m2 x e4m3 GEMM and the dgrad through the output block on the GPU.

Tolerances: the cast and its amax are integer / exact results (equality);
the GEMM against the fp64 product of the same fp8 operands: relative L2
<= 4e-3 and max|err| <= 1e-2 max|ref| (bf16 output); the FP8 dgrad against
the bf16 product: relative L2 <= 8e-2 (e5m2 keeps 2 mantissa bits), and the
same bound for the output block's dattn / du."""

import numpy as np
import pytest
import torch

from oracle import hstu_bwd_fp8_oracle as O

E5M2, E4M3 = torch.float8_e5m2, torch.float8_e4m3fn


def _rel(ref, got):
    ref, got = ref.double(), got.double()
    return float((got - ref).norm() / ref.norm().clamp_min(1e-30))


def test_oracle_cast_decode_bound_and_exact_powers():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(4096, generator=g) * torch.exp(torch.randn(4096, generator=g) * 3)
    for dtype, lim, mbits, sub in ((E5M2, 57344.0, 2, 2.0 ** -16), (E4M3, 448.0, 3, 2.0 ** -9)):
        inv = 0.37
        q, amax = O.cast_amax(x, inv, dtype, lim)
        v = (x * torch.tensor(inv, dtype=torch.float32)).clamp(-lim, lim).double()
        err = (q.double() - v).abs()
        assert bool((err <= torch.maximum(v.abs() * 2.0 ** -(mbits + 1), torch.tensor(sub / 2))).all())
        assert float(amax) == float(x.abs().max())
        p2 = torch.tensor([2.0 ** k for k in range(-6, 8)])
        qp, _ = O.cast_amax(p2, 1.0, dtype, lim)
        assert torch.equal(qp.double(), p2.double())


def test_oracle_published_scale_closed_form():
    for amax in (1e-3, 0.5, 7.25, 3e4):
        s = O.published_scale(amax, 8.0, 57344.0)
        assert abs(amax / s - 57344.0 / 8.0) <= 1e-3 * 57344.0 / 8.0
    assert O.published_scale(0.0, 8.0, 57344.0) > 0.0


def test_controller_warmup_publish_refresh(monkeypatch):
    """The delayed-scale policy on CPU tensors (the cast is the oracle's)."""
    import hstu_amd.bwd_fp8 as B

    cfg = B.Fp8BackwardConfig(enabled=True, warmup_calls=2, refresh_calls=3)
    monkeypatch.setattr(B, "quantize_row_major",
                        lambda v, inv, dtype=None, limit=None, partials=False: O.cast_amax(
                            v, float(inv.reshape(-1)[0]), dtype or E5M2, limit or 57344.0))
    B.reset_sites()
    g = [torch.full((4, 128), float(a)) for a in (2.0, 3.0, 1.0, 9.0, 4.0, 1.0)]
    assert B.quantize_gradient("site", g[0], config=cfg) is None
    assert B.quantize_gradient("site", g[1], config=cfg) is None      # warm-up ends: publish max(2, 3)
    st = B.find_site("site")
    s0 = O.published_scale(3.0, 8.0, 57344.0)
    assert st.live and float(st.scale) == pytest.approx(s0, rel=1e-6)
    q, dec = B.quantize_gradient("site", g[2], snapshot_decode_scale=True, config=cfg)   # call 3: refresh
    assert float(dec) == pytest.approx(s0, rel=1e-6)         # the scale it was cast with
    assert float(q.float()[0, 0]) * s0 == pytest.approx(1.0, rel=0.13)
    s1 = O.published_scale(1.0, 8.0, 57344.0)                 # window of call 3 only
    assert float(st.scale) == pytest.approx(s1, rel=1e-6)
    q4, dec4 = B.quantize_gradient("site", g[3], config=cfg)  # 9.0 > s1 * 57344 = 8: overflowed
    assert int(st.overflow_windows) == 1
    assert float(dec4) == pytest.approx(s1, rel=1e-6)
    _, dec5 = B.quantize_gradient("site", g[4], config=cfg)
    q6, dec6 = B.quantize_gradient("site", g[5], config=cfg)  # call 6: refresh, default decode = new scale
    assert float(dec6) == pytest.approx(O.published_scale(9.0, 8.0, 57344.0), rel=1e-6)
    assert B.quantize_gradient("site", g[0], config=B.Fp8BackwardConfig(enabled=False)) is None
    B.reset_sites()


def test_config_from_env_is_read_once(monkeypatch):
    """The reference's switch names set the process default when it is first
    used; later changes to the environment do not reach running calls."""
    import hstu_amd.bwd_fp8 as B

    monkeypatch.setenv("DLRM_HSTU_FP8_BWD", "1")
    monkeypatch.setenv("DLRM_HSTU_FP8_BWD_WARMUP_CALLS", "7")
    monkeypatch.setenv("DLRM_HSTU_FP8_BWD_GRAD_FORMAT", "e4m3")
    B.set_default_config(None)
    c = B.default_config()
    assert c.enabled and c.warmup_calls == 7 and c.grad_dtype == E4M3 and c.grad_limit == 448.0
    monkeypatch.setenv("DLRM_HSTU_FP8_BWD", "0")
    assert B.enabled()                                          # unchanged until re-read
    B.set_default_config(None)
    assert not B.enabled()
    with pytest.raises(ValueError):
        B.Fp8BackwardConfig(grad_format="e3m4")
    B.set_default_config(None)


def test_site_names_per_layer():
    import hstu_amd.bwd_fp8 as B

    B.reset_sites()
    assert B.site_name("output_projection", 111) == "output_projection.L0"
    assert B.site_name("output_projection", 222) == "output_projection.L1"
    assert B.site_name("output_projection", 111) == "output_projection.L0"
    assert B.site_name("x", None) == "x"
    B.reset_sites()


@pytest.mark.gpu
@pytest.mark.parametrize("src", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("dst,lim", [(E5M2, 57344.0), (E4M3, 448.0)])
def test_cast_amax_bit_exact(hip_lib, src, dst, lim):
    import hstu_amd.bwd_fp8 as B

    g = torch.Generator().manual_seed(3)
    n = 3 * 8192 + 96
    x = torch.randn(n, generator=g) * torch.exp(torch.randn(n, generator=g) * 4)
    x[:5] = torch.tensor([0.0, -0.0, 1e-30, 7e4, -9e4])   # zero, tiny, clipped both ways
    x = x.to(src)
    inv = torch.tensor([0.731], dtype=torch.float32)
    q, amax = B.quantize_row_major(x.cuda(), inv.cuda(), dtype=dst, limit=lim)
    wq, wamax = O.cast_amax(x, float(inv), dst, lim)
    assert torch.equal(q.cpu().view(torch.uint8), wq.view(torch.uint8))
    assert float(amax) == float(wamax)


@pytest.mark.gpu
def test_e5m2_gemm_against_fp64(hip_lib):
    import hstu_amd.bwd_fp8 as B

    g = torch.Generator().manual_seed(5)
    M, K, N = 300, 512, 1536
    dy = torch.randn(M, K, generator=g)
    w = torch.randn(N, K, generator=g) / K ** 0.5
    gs, ws = 1.0 / 4096, float(w.abs().max()) / 448
    g8 = (dy / gs).clamp(-57344, 57344).to(E5M2)
    w8 = (w / ws).to(E4M3)
    out = B.fp8_dgrad(g8.cuda(), torch.tensor([gs]).cuda(), w8.cuda(), torch.tensor([ws]).cuda())
    ref = O.dgrad(g8, gs, w8, ws)
    got = out.cpu().double()
    assert _rel(ref, got) <= 4e-3
    assert float((got - ref).abs().max()) <= 1e-2 * float(ref.abs().max())


@pytest.mark.gpu
def test_output_projection_dgrad_warmup_then_fp8(hip_lib, fp8_bwd):
    import hstu_amd.bwd_fp8 as B

    fp8_bwd(enabled=True)
    B.reset_sites()
    g = torch.Generator(device="cuda").manual_seed(7)
    w = (torch.randn(1536, 512, device="cuda", generator=g) / 40).requires_grad_(True)
    outs = []
    for i in range(6):
        dout = torch.randn(1000, 512, device="cuda", generator=g).to(torch.bfloat16)
        outs.append((dout, B.output_projection_dgrad(dout, w)))
    assert all(o is None for _, o in outs[:4])                 # 4 warm-up calls
    for dout, o in outs[4:]:
        ref = dout.double() @ w.detach().double().t()
        assert o.dtype == torch.bfloat16 and o.shape == (1000, 1536)
        assert _rel(ref, o) <= 8e-2
    # a non-parameter weight (a per-call copy) never engages
    assert B.output_projection_dgrad(outs[0][0], w.detach().clone()) is None
    B.reset_sites()


@pytest.mark.gpu
def test_output_block_backward_with_fp8_dgrad(hip_lib, fp8_bwd):
    import hstu_amd
    import hstu_amd.bwd_fp8 as B

    T, D = 2000, 512
    g = torch.Generator(device="cuda").manual_seed(11)
    attn = torch.randn(T, D, device="cuda", generator=g).to(torch.bfloat16)
    u = torch.randn(T, D, device="cuda", generator=g).to(torch.bfloat16)
    x = torch.randn(T, D, device="cuda", generator=g).to(torch.bfloat16)
    nw = torch.ones(D, device="cuda", dtype=torch.bfloat16)
    nb = torch.zeros(D, device="cuda", dtype=torch.bfloat16)
    W = (torch.randn(3 * D, D, device="cuda", generator=g) / 40).to(torch.bfloat16).requires_grad_(True)
    dout = torch.randn(T, D, device="cuda", generator=g).to(torch.bfloat16)

    def grads():
        a, uu = attn.clone().requires_grad_(True), u.clone().requires_grad_(True)
        out = hstu_amd.triton_hstu_compute_output(a, uu, x, nw, nb, W, 1e-6, 0.0, True, silu_u=True, concat_u=True,
                                                  concat_x=True, mul_u_activation_type="silu",
                                                  recompute_y_in_backward=True)
        out.backward(dout)
        return a.grad.float(), uu.grad.float()

    fp8_bwd(enabled=False)
    ref = grads()
    fp8_bwd(enabled=True)
    B.reset_sites()
    for _ in range(4):
        warm = grads()                                        # warm-up: bf16, identical
    assert torch.equal(warm[0], ref[0]) and torch.equal(warm[1], ref[1])
    fp8 = grads()
    for r, f in zip(ref, fp8):
        assert _rel(r, f) <= 8e-2
        assert not torch.equal(r, f)                          # the FP8 path ran
    B.reset_sites()


def test_oracle_colsum_closed_forms():
    M, N = 1000, 512
    c = torch.linspace(-3, 3, N).to(torch.bfloat16).float()
    x = c[None, :].expand(M, N).clone()
    x[:, :128] = torch.where(torch.arange(M)[:, None] % 2 == 0, 1.5, -1.5).expand(M, 128)
    out, amax, cs = O.cast_amax_colsum(x.to(torch.bfloat16), 0.5, E5M2, 57344.0, pad_to=128)
    assert out.shape == (1024, N) and out.dtype == E5M2
    assert bool((out[M:].view(torch.uint8) == 0).all())
    q, a = O.cast_amax(x.to(torch.bfloat16), 0.5, E5M2, 57344.0)
    assert torch.equal(out[:M].view(torch.uint8), q.view(torch.uint8)) and float(amax) == float(a)
    assert torch.equal(cs[:128], torch.zeros(128, dtype=torch.float64))      # alternating +-1.5, M even
    assert torch.equal(cs[128:], (c[128:] * M).double())                       # constant columns
    z, za, zc = O.cast_amax_colsum(torch.zeros(0, 256, dtype=torch.bfloat16), 1.0, E5M2, 57344.0, pad_to=128)
    assert z.shape == (0, 256) and float(za) == 0.0 and torch.equal(zc, torch.zeros(256, dtype=torch.float64))


def test_oracle_uvqk_backward_unquantized_is_autograd():
    """With unquantized operands (scale 1) the oracle's three gradients are
    those of z = x W + b (a transposed operand or a dropped term fails)."""
    g = torch.Generator().manual_seed(2)
    x = torch.randn(37, 64, generator=g, dtype=torch.float64, requires_grad=True)
    W = torch.randn(64, 256, generator=g, dtype=torch.float64, requires_grad=True)
    b = torch.randn(256, generator=g, dtype=torch.float64, requires_grad=True)
    dz = torch.randn(37, 256, generator=g, dtype=torch.float64)
    (x @ W + b).backward(dz)
    d_x, d_w, d_b = O.uvqk_backward(dz, x.detach(), dz, 1.0, W.detach(), 1.0)
    assert torch.allclose(d_x, x.grad) and torch.allclose(d_w, W.grad) and torch.allclose(d_b, b.grad)


def test_uvqk_controller_declines_and_snapshot(monkeypatch):
    """Host logic of uvqk_projection_backward on the CPU: declines, the
    warm-up, and the decode-scale snapshot on a refresh call (the cast, the
    weight cast and the GEMM are the oracle's)."""
    import hstu_amd.bwd_fp8 as B

    W = torch.randn(128, 256).to(torch.bfloat16).requires_grad_(True)
    dz = torch.randn(64, 256).to(torch.bfloat16)
    xn = torch.randn(64, 128).to(torch.bfloat16)
    assert B.uvqk_projection_backward(dz, xn, None, W, config=B.Fp8BackwardConfig()) is None   # off by default
    assert B.uvqk_projection_backward(dz, xn, None, W, config=B.Fp8BackwardConfig(
        uvqk=True, grad_format="e4m3")) is None                                               # needs e5m2
    cfg = B.Fp8BackwardConfig(uvqk=True, warmup_calls=2, refresh_calls=3)
    B.reset_sites()
    assert B.uvqk_projection_backward(dz, xn, None, W.detach(), config=cfg) is None    # not the leaf parameter
    assert B.uvqk_projection_backward(dz[:, :200].contiguous(), xn, None, W[:, :200], config=cfg) is None  # N % 256
    assert B.uvqk_projection_backward(dz, None, None, W, config=cfg) is None           # no normed_x at all
    assert not B._registry.sites                                               # declines touch no state
    seen = []

    def cast(v, inv, pad_to=1, out=None, dtype=None):
        q, a, cs = O.cast_amax_colsum(v, float(inv.reshape(-1)[0]), E5M2, 57344.0, pad_to)
        return q, a.float(), cs.float()

    def gemm(g8, gs, w8, ws, out_dtype=torch.bfloat16):
        seen.append(float(gs.reshape(-1)[0]))
        return O.dgrad(g8, float(gs.reshape(-1)[0]), w8, float(ws.reshape(-1)[0])).to(out_dtype)

    monkeypatch.setattr(B, "quantize_amax_colsum", cast)
    monkeypatch.setattr(B, "quantize_weight", lambda w: (
        (w.float() / O.weight_scale(w)).to(E4M3), O.weight_scale(w)))
    monkeypatch.setattr(B, "fp8_dgrad", gemm)
    amaxes = [2.0, 3.0, 1.0, 5.0]
    outs = []
    for a in amaxes:
        d = dz.float() / dz.float().abs().max() * a
        outs.append(B.uvqk_projection_backward(d.to(torch.bfloat16), None, None, W, recompute_normed_x=lambda: xn,
                                               config=cfg))
    assert outs[0] is None and outs[1] is None                                  # warm-up
    s0 = O.published_scale(3.0, 8.0, 57344.0)
    assert seen[0] == pytest.approx(s0, rel=1e-6)                              # call 3 decodes with the cast's scale
    assert seen[1] == pytest.approx(O.published_scale(1.0, 8.0, 57344.0), rel=1e-6)  # refreshed after call 3
    d_x, d_w, d_b = outs[2]
    assert d_w.shape == (128, 256) and d_b.dtype == torch.float32 and d_x.shape == (64, 128)
    B.reset_sites()


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,pad,ld", [(1000, 2048, 1, 2048), (513, 512, 128, 512), (1, 256, 128, 264),
                                        (0, 256, 128, 256), (3 * 512 + 7, 768, 1, 768)])
@pytest.mark.parametrize("dst", [E5M2, E4M3])
def test_cast_amax_colsum_bit_exact(hip_lib, M, N, pad, ld, dst):
    """Payload and amax equal to the oracle's; rows past M zero; colsum within
    the fp32 summation bound of the float64 sum."""
    import hstu_amd.bwd_fp8 as B

    g = torch.Generator().manual_seed(M + N)
    base = torch.randn(M, ld, generator=g) * torch.exp(torch.randn(M, ld, generator=g) * 2)
    if M > 3:
        base[:3, :3] = torch.tensor([[0.0, 7e4, -9e4], [1e-30, -0.0, 3.0], [2.0 ** -20, 1.0, -1.0]])
    x = base.to(torch.bfloat16)[:, :N]                                          # row stride ld
    inv = torch.tensor([0.37], dtype=torch.float32)
    lim = 57344.0 if dst == E5M2 else 448.0
    xd = x.cuda() if ld == N else base.to(torch.bfloat16).cuda()[:, :N]
    q, amax, cs = B.quantize_amax_colsum(xd, inv.cuda(), pad_to=pad, dtype=dst)
    wq, wamax, wcs = O.cast_amax_colsum(x, float(inv), dst, lim, pad_to=pad)
    assert q.shape == wq.shape
    assert torch.equal(q.cpu().view(torch.uint8), wq.view(torch.uint8))
    assert float(amax) == float(wamax)
    stripes = (M + 511) // 512
    bound = (72 + stripes) * 2.0 ** -24 * x.double().abs().sum(0) + 1e-30
    assert bool(((cs.cpu().double() - wcs).abs() <= bound).all())


@pytest.mark.gpu
def test_uvqk_projection_backward_warmup_then_fp8(hip_lib, fp8_bwd):
    import hstu_amd.bwd_fp8 as B

    fp8_bwd(uvqk=True)
    B.reset_sites()
    g = torch.Generator(device="cuda").manual_seed(9)
    W = (torch.randn(512, 2048, device="cuda", generator=g) / 25).to(torch.bfloat16).requires_grad_(True)
    res = []
    for i in range(6):
        dz = torch.randn(1000, 2048, device="cuda", generator=g).to(torch.bfloat16)
        xn = torch.randn(1000, 512, device="cuda", generator=g).to(torch.bfloat16)
        res.append((dz, xn, B.uvqk_projection_backward(dz, xn, None, W)))
    assert all(r is None for _, _, r in res[:4])
    st = B.find_site("uvqk_projection", layer=0)
    for dz, xn, r in res[4:]:
        d_x, d_w, d_b = r
        assert d_x.dtype == torch.bfloat16 and d_x.shape == (1000, 512)
        ref_x = dz.double() @ W.detach().double().t()
        assert _rel(ref_x, d_x) <= 8e-2
        # against the same quantized operands: the GEMM's accumulation only
        dz8, _, cs = O.cast_amax_colsum(dz.cpu(), float(st.inv_scale), E5M2, 57344.0)
        w8, ws = (W.detach().float().cpu() / O.weight_scale(W.cpu())).to(E4M3), O.weight_scale(W.cpu())
        rx, rw, rb = O.uvqk_backward(dz, xn, dz8, float(st.scale), w8, float(ws))
        assert _rel(rx, d_x.cpu()) <= 4e-3
        assert _rel(rw, d_w.cpu()) <= 1e-2
        assert _rel(rb, d_b.cpu()) <= 1e-5
    B.reset_sites()


def test_oracle_wgrad_closed_forms():
    g = torch.Generator().manual_seed(4)
    b = torch.randn(50, 24, generator=g)
    assert torch.allclose(O.wgrad(torch.ones(50, 3), b), b.double().sum(0)[None, :].expand(3, 24))
    a = torch.randn(50, 7, generator=g)
    hot = torch.zeros(50, 5)
    hot[torch.arange(5) * 3, torch.arange(5)] = 1.0                        # token 3c -> column c
    assert torch.allclose(O.wgrad(a, hot, 2.0, 0.5), a.double()[torch.arange(5) * 3].t())


@pytest.mark.gpu
@pytest.mark.parametrize("shape,dtype,zero", [((1536, 512), torch.bfloat16, False), ((512, 2048), torch.bfloat16, False),
                                              ((256, 96), torch.float32, False), ((128, 64), torch.bfloat16, True)])
def test_quantize_weight_two_launches_bitwise(hip_lib, shape, dtype, zero):
    """hstu_quantize_e4m3_unit (block maxima, then scale + cast in one
    launch) equals the torch expression it replaces bit for bit: scale =
    amax.clamp_min(1e-30) / 448 and the cast at 1 / scale (an all-zero weight
    takes the clamp)."""
    import hstu_amd.bwd_fp8 as B

    g = torch.Generator(device="cuda").manual_seed(sum(shape))
    w = (torch.randn(shape, device="cuda", generator=g) * 0.05).to(dtype)
    if zero:
        w.zero_()
    q, s = B.quantize_weight(w)
    amax = w.abs().amax().float().clamp_min(1.0e-30)
    s_ref = (amax / B.E4M3_MAX).reshape(1)
    q_ref, _ = B.quantize_row_major(w, 1.0 / s_ref, dtype=E4M3, limit=B.E4M3_MAX)
    assert torch.equal(s, s_ref)
    assert torch.equal(q.view(torch.uint8), q_ref.view(torch.uint8))


@pytest.mark.gpu
def test_site_update_matches_the_policy_steps(hip_lib):
    """hstu_fp8_site_update (one launch) against GradScaleSite's own torch
    steps (fold, snapshot, roll) on a copy of the state, over a sequence of
    calls: warm-up, publish, overflow, refresh with and without a snapshot;
    states and snapshots bitwise equal."""
    import hstu_amd.bwd_fp8 as B

    cfg = B.Fp8BackwardConfig(enabled=True)
    a = B.GradScaleSite(torch.device("cuda"))
    b = B.GradScaleSite(torch.device("cuda"))
    g = torch.Generator(device="cuda").manual_seed(5)
    seq = [(0.5, False, False), (3.0, True, False), (1.0, False, True), (1e6, False, False), (0.25, True, True),
           (7.0, False, False), (0.0, True, False)]
    for peak, roll, snap in seq:
        parts = torch.rand(37, device="cuda", generator=g) * peak
        got = a.update(parts, cfg, roll=roll, snapshot=snap)
        b.fold(parts.amax(), cfg)
        want = b.scale.clone() if snap else None
        if roll:
            b.roll(cfg)
        assert torch.equal(a.state, b.state) and a.live == b.live
        assert (got is None) == (want is None) and (got is None or torch.equal(got, want))
    assert int(a.overflow_windows) >= 1
