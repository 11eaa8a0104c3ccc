"""GPU parity of ``hstu_compute_uqvk`` and the unfused (prefill) branch of
``hstu_preprocess_and_attention`` on this build's kernels (``kernel=TRITON``):
the LayerNorm kernel, the bf16 projection GEMM, the token-axis weight
gradient and the LayerNorm backward (reference ``ops/hstu_compute.py:86-144,
290-433``).

Small sizes: against the float64 composition ``F.layer_norm`` -> ``addmm``
-> split -> ``silu`` (the reference's PyTorch path) on the same bf16 inputs,
forward and backward: relative L2 <= 1e-2 for every output and gradient,
``assert_close(rtol=1e-2, atol=1e-2)`` for the row-wise ones (u, q, k, v,
dx), and max|err| <= 2e-2 max|ref| for the parameter gradients (sums over
the tokens of bf16 products).  Config 2 and config 3 token counts: against the same composition
in float32 on the device, relative L2 <= 1e-2 for u, q, k, v and every
gradient.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import hstu_layer_oracle as LO
from oracle import hstu_oracle as orc

pytestmark = pytest.mark.gpu
DEV = "cuda"
H, D = 4, 128


def _rel_l2(ref, got):
    ref, got = ref.double(), got.double()
    return float((got - ref).norm() / ref.norm().clamp_min(1e-30))


def _ref_uqvk(x, nw, nb, W, b):
    xn = F.layer_norm(x, (x.shape[1],), nw, nb, 1e-6)
    uvqk = torch.addmm(b, xn, W)
    u, v, q, k = torch.split(uvqk, [H * D] * 4, dim=1)
    return F.silu(u), q.reshape(-1, H, D), k.reshape(-1, H, D), v.reshape(-1, H, D)


def _inputs(T, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, 512, generator=g).to(torch.bfloat16)
    p = LO.make_layer_params(512, seed=seed + 1)
    outs = [torch.randn(T, H * D, generator=g).to(torch.bfloat16)] + [
        torch.randn(T, H, D, generator=g).to(torch.bfloat16) for _ in range(3)]
    return x, p["input_norm_weight"], p["input_norm_bias"], p["uvqk_weight"], p["uvqk_bias"], outs


def _run(fn, x, nw, nb, W, b, douts):
    leaves = [t.requires_grad_(True) for t in (x, nw, nb, W, b)]
    outs = fn(*leaves)
    torch.autograd.backward(list(outs), list(douts))
    return [o.detach() for o in outs], [t.grad for t in leaves]


@pytest.mark.parametrize("T", [1, 300, 1029])
def test_uqvk_small_vs_oracle(hip_lib, T):
    from hstu_amd import HammerKernel
    from hstu_amd.hstu_preprocess import hstu_compute_uqvk

    x, nw, nb, W, b, douts = _inputs(T, 11)
    got_o, got_g = _run(lambda *a: hstu_compute_uqvk(a[0], a[1], a[2], 1e-6, H, D, D, a[3], a[4],
                                                     kernel=HammerKernel.TRITON),
                        *(t.to(DEV) for t in (x, nw, nb, W, b)), [t.to(DEV) for t in douts])
    ref_o, ref_g = _run(_ref_uqvk, *(t.double() for t in (x, nw, nb, W, b)), [t.double() for t in douts])
    for name, r, g in zip(("u", "q", "k", "v", "dx", "dnorm_w", "dnorm_b", "dW", "db"), ref_o + ref_g,
                          got_o + got_g):
        g = g.double().cpu()
        if name in ("u", "q", "k", "v", "dx"):
            torch.testing.assert_close(g, r, rtol=1e-2, atol=1e-2, msg=name)
        else:  # sums over the tokens of bf16 products: relative to the largest entry
            assert float((g - r).abs().max()) <= 2e-2 * float(r.abs().max()), name
        if r.norm() > 0:
            assert _rel_l2(r, g) <= 1e-2, name


@pytest.mark.parametrize("cfg", [2, 3])
def test_uqvk_config_tokens(hip_lib, cfg):
    from hstu_amd import HammerKernel
    from hstu_amd.hstu_preprocess import hstu_compute_uqvk

    T = int(orc.lengths_for_config(cfg).sum())
    print(f"uqvk config {cfg}: T={T}", flush=True)
    x, nw, nb, W, b, douts = (t if isinstance(t, list) else t.to(DEV) for t in _inputs(T, 5))
    douts = [t.to(DEV) for t in douts]
    got_o, got_g = _run(lambda *a: hstu_compute_uqvk(a[0], a[1], a[2], 1e-6, H, D, D, a[3], a[4],
                                                     kernel=HammerKernel.TRITON), x, nw, nb, W, b, douts)
    ref_o, ref_g = _run(_ref_uqvk, *(t.detach().float() for t in (x, nw, nb, W, b)), [t.float() for t in douts])
    for name, r, g in zip(("u", "q", "k", "v", "dx", "dnorm_w", "dnorm_b", "dW", "db"), ref_o + ref_g,
                          got_o + got_g):
        e = _rel_l2(r, g.float())
        assert e <= 1e-2, f"{name} rel L2 {e:.3e}"


def test_prefill_branch_runs_hip_attention(hip_lib):
    """``hstu_preprocess_and_attention(prefill=True, kernel=TRITON)`` takes
    the unfused branch: the kernel-backed uqvk and the HIP attention, equal
    to the float64 composition of the reference's PyTorch path."""
    from hstu_amd import HammerKernel
    from hstu_amd.hstu_preprocess import hstu_preprocess_and_attention

    lengths = np.array([100, 7, 256, 33])
    T, N = int(lengths.sum()), 256
    x, nw, nb, W, b, _ = _inputs(T, 21)
    offs = orc.offsets_from_lengths(lengths)
    u, attn, k, v = hstu_preprocess_and_attention(
        x.to(DEV), nw.to(DEV), nb.to(DEV), 1e-6, H, D, D, W.to(DEV), b.to(DEV), N, offs.to(DEV), D ** -0.5, True,
        None, 0, 0, False, False, False, prefill=True, kernel=HammerKernel.TRITON)
    ur, qr, kr, vr = _ref_uqvk(*(t.double() for t in (x, nw, nb, W, b)))
    # the attention's inputs are the kernel path's bf16 q/k/v
    qb, kb, vb = (t.to(torch.bfloat16).double() for t in (qr, kr, vr))
    ar = orc.hstu_mha_dense(N, D ** -0.5, qb, kb, vb, offs, dtype=torch.float64).reshape(T, H * D)
    assert _rel_l2(ur, u.cpu()) <= 1e-2
    assert _rel_l2(kr, k.cpu()) <= 1e-2 and _rel_l2(vr, v.cpu()) <= 1e-2
    e = _rel_l2(ar, attn.float().cpu())
    assert e <= 1e-2, f"attn rel L2 {e:.3e}"
