"""GPU parity of the delta-q (targets-only / cached) attention through the HIP
C ABI against the float64 oracle ``cached_hstu_mha`` (itself pinned to the
last rows of the full attention and, for the backward, to the full
attention's backward with dO zero outside those rows).

Tolerances: bf16 ``assert_close(rtol=1e-2, atol=1e-2)`` plus relative L2 <=
1e-2; e4m3 k / v (per-tensor scales) relative L2 <= 1.5e-2 against the
dequantized inputs.  Outputs are bitwise deterministic (fixed-order chunk
sums), which the config-3 test checks through sub-batch independence.
"""

import numpy as np
import pytest
import torch

from oracle import hstu_oracle as orc

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _ops():
    import hstu_amd

    return hstu_amd


def _rel(ref, got):
    ref, got = ref.double(), got.double()
    return float((got - ref).norm() / ref.norm().clamp_min(1e-30))


def _case(lengths, H, D, ds, seed, fp8, std=0.5):
    q, k, v = orc.make_qkv(lengths, H, D, std, seed=seed)
    offs = orc.offsets_from_lengths(lengths)
    rows = torch.cat([torch.arange(int(offs[b + 1]) - ds, int(offs[b + 1])) for b in range(len(lengths))])
    qd = q[rows].contiguous()
    if fp8:
        (q8, sq), (k8, sk), (v8, sv) = (orc.quantize_e4m3_per_tensor(x) for x in (qd, k, v))
        deq = [x8.float() * float(s) for x8, s in ((q8, sq), (k8, sk), (v8, sv))]
        return offs, rows, (q8, k8, v8), tuple(float(s) for s in (sq, sk, sv)), deq
    qd, k, v = (x.to(torch.bfloat16) for x in (qd, k, v))
    return offs, rows, (qd, k, v), (1.0, 1.0, 1.0), [x.float() for x in (qd, k, v)]


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("ds,nt,ctx,win", [(1, None, 0, 0), (2, None, 0, 0), (1, [1, 3, 1, 2], 0, 0),
                                           (3, None, 5, 40)])
def test_delta_fwd(hip_lib, fp8, ds, nt, ctx, win):
    ops = _ops()
    lengths = [300, 17, 600, 129]
    H, D, N = 4, 128, 640
    offs, rows, (qd, k, v), (sq, sk, sv), deq = _case(lengths, H, D, ds, 1, fp8)
    num_targets = None if nt is None else torch.tensor(nt, dtype=torch.int32)
    out = ops.triton_cached_hstu_mha(N, 0.125, qd.to(DEV), k.to(DEV), v.to(DEV), offs.to(DEV),
                                     None if nt is None else num_targets.to(DEV), win, ctx,
                                     q_scale=sq, k_scale=sk, v_scale=sv)
    ref = orc.cached_hstu_mha(N, 0.125, deq[0].double(), deq[1].double(), deq[2].double(), offs,
                              num_targets=num_targets, max_attn_len=win, contextual_seq_len=ctx)
    got = out.float().cpu()
    if fp8:
        assert _rel(ref, got) <= 1.5e-2
    else:
        torch.testing.assert_close(got, ref.float(), rtol=1e-2, atol=1e-2)
        assert _rel(ref, got) <= 1e-2


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("ds", [1, 2, 3, 4])
def test_delta_bwd(hip_lib, fp8, ds):
    ops = _ops()
    lengths = [300, 17, 600, 129, 1000]
    H, D, N = 4, 128, 1000
    offs, rows, (qd, k, v), (sq, sk, sv), deq = _case(lengths, H, D, ds, 2, fp8)
    dout = torch.randn(qd.shape, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
    dq = torch.empty(qd.shape, dtype=torch.bfloat16, device=DEV)
    dk = torch.full(k.shape, 7.0, dtype=torch.bfloat16, device=DEV)  # every row must be overwritten
    dv = torch.full(v.shape, 7.0, dtype=torch.bfloat16, device=DEV)
    ops.triton_hstu_attention_delta_bwd(dout.to(DEV), qd.to(DEV), k.to(DEV), v.to(DEV), dq, dk, dv, offs.to(DEV), N,
                                        0.125, sk, sv, q_scale=sq)
    args = [x.double().requires_grad_(True) for x in deq]
    orc.cached_hstu_mha(N, 0.125, *args, offs).backward(dout.double())
    tol = 1.5e-2 if fp8 else 1e-2
    for name, ref, got in (("dq", args[0].grad, dq), ("dk", args[1].grad, dk), ("dv", args[2].grad, dv)):
        assert _rel(ref, got.float().cpu()) <= tol, (name, _rel(ref, got.float().cpu()))
        if not fp8:
            torch.testing.assert_close(got.float().cpu(), ref.float(), rtol=1e-2, atol=1e-2, msg=name)


def test_delta_mha_autograd_and_pytorch_backend(hip_lib):
    ops = _ops()
    lengths = [40, 90, 7]
    H, D, N = 2, 64, 96
    offs, rows, (qd, k, v), _, deq = _case(lengths, H, D, 1, 3, False)
    a = [x.to(DEV).requires_grad_(True) for x in (qd, k, v)]
    out = ops.delta_hstu_mha(N, 0.2, a[0], a[1], a[2], offs.to(DEV), kernel=ops.HammerKernel.TRITON)
    ref = ops.delta_hstu_mha(N, 0.2, *(x.to(DEV).float() for x in (qd, k, v)), offs.to(DEV))  # PYTORCH backend
    torch.testing.assert_close(out.float(), ref, rtol=1e-2, atol=1e-2)
    g = torch.randn(out.shape, device=DEV).to(torch.bfloat16)
    out.backward(g)
    b = [x.to(DEV).float().requires_grad_(True) for x in (qd, k, v)]
    ops.delta_hstu_mha(N, 0.2, b[0], b[1], b[2], offs.to(DEV)).backward(g.float())
    for x, y in zip(a, b):
        assert _rel(y.grad, x.grad.float()) <= 1e-2


def test_delta_config3_targets_only(hip_lib):
    """BASELINE config 3's sequences (B = 128 Zipf lengths, T = 162 251, N =
    4096, H = 4, D = 128, e4m3 k / v) with one target per sequence: the oracle
    on a sample incl. the longest sequence, and bitwise sub-batch independence."""
    ops = _ops()
    lengths = orc.lengths_for_config(3)
    H, D, N = 4, 128, 4096
    offs, rows, (qd, k, v), (sq, sk, sv), deq = _case(lengths, H, D, 1, 5, True, std=1.0)
    dout = torch.randn(qd.shape, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)

    def run(lens, q_, k_, v_, do_):
        o = orc.offsets_from_lengths(lens).to(DEV)
        out = ops.triton_cached_hstu_mha(N, 1 / D ** 0.5, q_.to(DEV), k_.to(DEV), v_.to(DEV), o, q_scale=sq,
                                         k_scale=sk, v_scale=sv)
        dq = torch.empty(q_.shape, dtype=torch.bfloat16, device=DEV)
        dk = torch.empty(k_.shape, dtype=torch.bfloat16, device=DEV)
        dv = torch.empty(v_.shape, dtype=torch.bfloat16, device=DEV)
        ops.triton_hstu_attention_delta_bwd(do_.to(DEV), q_.to(DEV), k_.to(DEV), v_.to(DEV), dq, dk, dv, o, N,
                                            1 / D ** 0.5, sk, sv, q_scale=sq)
        return out.cpu(), dq.cpu(), dk.cpu(), dv.cpu()

    full = run(lengths, qd, k, v, dout)
    order = np.argsort(lengths)
    sample = sorted({int(order[-1]), int(order[0]), int(order[len(order) // 2])})
    krows = torch.cat([torch.arange(int(offs[b]), int(offs[b + 1])) for b in sample])
    sb = torch.tensor(sample)
    sub = run(lengths[sample], qd[sb], k[krows], v[krows], dout[sb])
    for name, a, b, sel in (("out", full[0], sub[0], sb), ("dq", full[1], sub[1], sb), ("dk", full[2], sub[2], krows),
                            ("dv", full[3], sub[3], krows)):
        assert torch.equal(a[sel], b), name
    so = orc.offsets_from_lengths(lengths[sample])
    args = [deq[0][sb].double().requires_grad_(True), deq[1][krows].double().requires_grad_(True),
            deq[2][krows].double().requires_grad_(True)]
    ref = orc.cached_hstu_mha(N, 1 / D ** 0.5, *args, so)
    ref.backward(dout[sb].double())
    assert _rel(ref.detach(), sub[0].float()) <= 1.5e-2
    for name, r, got in (("dq", args[0].grad, sub[1]), ("dk", args[1].grad, sub[2]), ("dv", args[2].grad, sub[3])):
        assert _rel(r, got.float()) <= 1.5e-2, name
