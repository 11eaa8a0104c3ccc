"""The full-FP8 backward's dO block quantizer: the oracle pinned on the CPU
(bit formula vs brute force, group layout, decode error), and the HIP kernel
bit-exact against it on the GPU (e4m3 bytes and E8 bytes are integer
results: equality is the bar)."""

import numpy as np
import pytest
import torch

from oracle import hstu_do_fp8_oracle as Q
from oracle import hstu_oracle as orc


def _amax_samples():
    rng = np.random.default_rng(0)
    vals = list(np.exp(rng.uniform(-60, 60, 4000)).astype(np.float32))
    for k in range(-70, 70):
        for m in (1.0, 1.25, 1.5, 1.75, 1.875, 1.999):
            vals.append(np.float32(m * 2.0 ** k))
    base = np.array([1.75 * 2.0 ** k for k in range(-40, 40)], dtype=np.float32)
    vals += list(np.nextafter(base, np.float32(np.inf)))
    vals += list(np.nextafter(base, np.float32(0)))
    vals += [np.float32(0.0), np.float32(1e-42), np.finfo(np.float32).tiny, np.float32(3e38), np.float32(448.0)]
    return np.array(vals, dtype=np.float32)


def test_group_exp_matches_brute_force():
    a = _amax_samples()
    got = Q.group_exp(a)
    want = np.array([Q.group_exp_brute(float(x)) for x in a])
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(float(a[i]), int(got[i]), int(want[i])) for i in bad[:5]]


def test_group_exp_range():
    a = _amax_samples()
    e = Q.group_exp(a)
    normal = (a >= np.finfo(np.float32).tiny) & (e > -60) & (e < 60)
    prod = a[normal].astype(np.float64) * 2.0 ** e[normal]
    assert np.all(prod > 224.0) and np.all(prod <= 448.0)
    assert Q.group_exp(np.float32(1.0)) == 8 and Q.group_exp(np.float32(1.75)) == 8
    assert Q.group_exp(np.nextafter(np.float32(1.75), np.float32(2))) == 7


def test_group_layout():
    p = np.arange(256)
    tile, half = Q.group_of(p)
    for t in range(4):
        for h in (0, 1):
            assert np.sum((tile == t) & (half == h)) == 32
    # constant on each aligned run of 8 tokens
    assert np.all(half.reshape(-1, 8) == half.reshape(-1, 8)[:, :1])
    assert list(half[:16]) == [0] * 8 + [1] * 8


def test_oracle_decodes_within_half_step_and_group_max():
    lengths = np.array([70, 5, 130, 64])
    offs = orc.offsets_from_lengths(lengths)
    g = torch.Generator().manual_seed(1)
    T, H, D = int(lengths.sum()), 4, 128
    x = (torch.randn(T, H, D, generator=g) * torch.exp(torch.randn(T, 1, 1, generator=g) * 3)).to(torch.bfloat16)
    y, e8 = Q.quantize_do_e4m3_blk(x, offs, 130)
    e = 127 - e8.numpy().astype(np.int64)
    dec = y.view(torch.float8_e4m3fn).float().numpy() * 2.0 ** (-e[:, :, None])
    xf = x.float().numpy()
    scaled = np.abs(xf) * 2.0 ** e[:, :, None]
    # half an e4m3 step: 2^-4 relative for normals, 2^-10 absolute below 2^-6
    tol = np.maximum(scaled / 16.0, 2.0 ** -10) * 2.0 ** (-e[:, :, None])
    assert np.all(np.abs(dec - xf) <= tol * 1.0001)
    # brute-force group maxima: every group's largest |x| * 2^e lands in (224, 448]
    for b in range(len(lengths)):
        st, L = int(offs[b]), int(lengths[b])
        for p0 in range(0, L, 64):
            for half in (0, 1):
                rows = [st + p for p in range(p0, min(L, p0 + 64)) if (p % 16) // 8 == half]
                if not rows:
                    continue
                for h in range(H):
                    am = np.abs(xf[rows, h]).max()
                    ee = set(e[rows, h].tolist())
                    assert len(ee) == 1
                    if am > 0:
                        assert 224.0 < am * 2.0 ** ee.pop() <= 448.0


def _case(lengths, H, D, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    T = int(np.sum(lengths))
    x = torch.randn(T, H, D, generator=g) * torch.exp(torch.randn(T, H, 1, generator=g) * 4)
    if T > 10:
        x[3:9] = 0.0                                  # an all-zero run
        x[9, 0] = 1e-40 if dtype == torch.float32 else 1e-38  # tiny values
    return x.to(dtype)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("H,D", [(4, 128), (8, 64), (2, 128), (2, 64), (1, 128)])
def test_do_blk_kernel_bit_exact(hip_lib, dtype, H, D):
    import hstu_amd

    lengths = np.array([200, 1, 64, 63, 129, 17, 300])
    N = 300
    offs = orc.offsets_from_lengths(lengths)
    x = _case(lengths, H, D, 7, dtype)
    y, e8 = hstu_amd.quantize_do_e4m3_blk(x.cuda(), offs.cuda(), N)
    wy, we8 = Q.quantize_do_e4m3_blk(x, offs, N)
    assert torch.equal(e8.cpu(), we8)
    assert torch.equal(y.cpu().view(torch.uint8), wy)


@pytest.mark.gpu
def test_do_blk_kernel_config3_strided(hip_lib):
    """Config 3's sequences at full size, dO read from a strided view."""
    import hstu_amd

    lengths = orc.lengths_for_config(3)
    offs = orc.offsets_from_lengths(lengths)
    T = int(np.sum(lengths))
    g = torch.Generator(device="cuda").manual_seed(3)
    big = torch.randn(T, 1024, device="cuda", generator=g).to(torch.bfloat16)
    x = big[:, 256:768].view(T, 4, 128)
    y, e8 = hstu_amd.quantize_do_e4m3_blk(x, offs.cuda(), 4096)
    # exact decode property on the whole tensor, oracle bytes on a sample of sequences
    e = 127 - e8.to(torch.int32)
    dec = y.float() * torch.exp2(-e.float())[:, :, None]
    xf = x.float()
    scaled = xf.abs() * torch.exp2(e.float())[:, :, None]
    tol = torch.clamp(scaled / 16, min=2.0 ** -10) * torch.exp2(-e.float())[:, :, None]
    assert bool(((dec - xf).abs() <= tol * 1.0001).all())
    for b in (0, int(np.argmax(lengths)), 77):
        st, en = int(offs[b]), int(offs[b + 1])
        so = torch.tensor([0, en - st])
        wy, we8 = Q.quantize_do_e4m3_blk(x[st:en].cpu(), so, 4096)
        assert torch.equal(e8[st:en].cpu(), we8)
        assert torch.equal(y[st:en].cpu().view(torch.uint8), wy)


def test_oracle_dequantize_exact_and_round_trip():
    from oracle import hstu_do_fp8_oracle as DO

    g = torch.Generator().manual_seed(12)
    lengths = [70, 5, 128]
    T = sum(lengths)
    offs = torch.tensor(np.concatenate([[0], np.cumsum(lengths)]))
    x = (torch.randn(T, 2, 128, generator=g) * torch.exp(torch.randn(T, 2, 1, generator=g) * 3)).to(torch.bfloat16)
    y, e8 = DO.quantize_do_e4m3_blk(x, offs, 128)
    d = DO.dequantize_do_e4m3_blk(y, e8)
    exact = y.view(torch.float8_e4m3fn).double() * torch.pow(2.0, e8.double() - 127.0)[:, :, None]
    assert torch.equal(d.double(), exact)                                   # no rounding in bf16
    xf = x.double()
    # half an e4m3 step: relative 2^-4 for normals, 2^-10 of the group's scale 2^-e for subnormals
    step = torch.pow(2.0, e8.double() - 127.0)[:, :, None] * 2.0 ** -10
    assert bool(((d.double() - xf).abs() <= xf.abs() * 2.0 ** -4 + step).all())


@pytest.mark.gpu
def test_dequantize_bit_exact(hip_lib):
    import hstu_amd

    lengths = [200, 64, 1, 333]
    T = sum(lengths)
    offs = torch.tensor(np.concatenate([[0], np.cumsum(lengths)]))
    g = torch.Generator().manual_seed(21)
    x = (torch.randn(T, 4, 128, generator=g) * torch.exp(torch.randn(T, 4, 1, generator=g) * 4)).to(torch.bfloat16)
    y, e8 = hstu_amd.quantize_do_e4m3_blk(x.cuda(), offs.cuda(), 512)
    d = hstu_amd.dequantize_do_e4m3_blk(y, e8)
    want = Q.dequantize_do_e4m3_blk(y.cpu(), e8.cpu())
    assert torch.equal(d.cpu().view(torch.int16), want.view(torch.int16))
