"""Host-side logic on the CPU: shape policy and fallible entry points, the
PYTORCH backend against the oracle, bench CLI guard."""

import subprocess
import sys
from pathlib import Path

import pytest
import torch

from oracle import hstu_oracle as orc

REPO = Path(__file__).resolve().parents[1]


def test_unsupported_shape_reasons():
    from hstu_amd import unsupported_shape_reason

    bf = torch.zeros(4, 2, 128, dtype=torch.bfloat16)
    assert "GPU" in unsupported_shape_reason(bf, bf, bf)
    assert "head dim" in unsupported_shape_reason(*(torch.zeros(4, 2, 96, dtype=torch.bfloat16),) * 3)
    assert "dtype" in unsupported_shape_reason(*(torch.zeros(4, 2, 128),) * 3)
    assert "d_v" in unsupported_shape_reason(bf, bf, torch.zeros(4, 2, 64, dtype=torch.bfloat16))
    f8 = torch.zeros(4, 2, 64, dtype=torch.float8_e4m3fn)
    assert "e4m3 head dim" in unsupported_shape_reason(f8, f8, f8)
    assert "num_softmax_heads" in unsupported_shape_reason(bf, bf, bf, num_softmax_heads=1)


def test_try_entry_points_decline_without_touching_outputs():
    from hstu_amd import try_hstu_attention_bwd, try_hstu_attention_fwd

    q = torch.zeros(4, 2, 128, dtype=torch.bfloat16)
    offs = torch.tensor([0, 4])
    assert try_hstu_attention_fwd(q=q, k=q, v=q, seq_offsets=offs, num_targets=None, N=4, alpha=0.1,
                                  max_attn_len=0, contextual_seq_len=0) is None
    dq = torch.full_like(q, 3.0)
    assert try_hstu_attention_bwd(dout=q, q=q, k=q, v=q, dq=dq, dk=dq, dv=dq, seq_offsets=offs, num_targets=None,
                                  N=4, alpha=0.1, max_attn_len=0, contextual_seq_len=0) is False
    assert torch.all(dq == 3.0)


def test_kernel_ops_raise_instead_of_falling_back():
    from hstu_amd import triton_hstu_attention_fwd

    q = torch.zeros(4, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError):
        triton_hstu_attention_fwd(4, 0.1, q, q, q, torch.tensor([0, 4]), None, 0, 0, None, False, 0)


@pytest.mark.parametrize("kw", [{}, {"num_targets": torch.tensor([2, 1])}, {"max_attn_len": 3},
                                {"contextual_seq_len": 2}])
def test_pytorch_backend_matches_oracle(kw):
    """kernel=PYTORCH (the reference's default backend) restated with torch ops."""
    from hstu_amd import HammerKernel, hstu_mha

    lengths = [7, 4]
    q, k, v = orc.make_qkv(lengths, 2, 8, 0.6, seed=3, dtype=torch.float64)
    offs = orc.offsets_from_lengths(lengths)
    got = hstu_mha(8, 0.3, q, k, v, offs, kernel=HammerKernel.PYTORCH, **kw)
    want = orc.hstu_mha_dense(8, 0.3, q, k, v, offs, kw.get("num_targets"), kw.get("max_attn_len", 0),
                              kw.get("contextual_seq_len", 0), dtype=torch.float64)
    assert torch.allclose(got, want, atol=1e-12)


def test_pytorch_backend_bias_and_autograd():
    from hstu_amd import HammerKernel, hstu_mha

    lengths = [5, 6]
    q, k, v = orc.make_qkv(lengths, 2, 4, 0.6, seed=4, dtype=torch.float64)
    offs = orc.offsets_from_lengths(lengths)
    bias = orc.make_bias(2, 3, seed=1, std=0.4).double()
    got = hstu_mha(6, 0.5, q, k, v, offs, kernel=HammerKernel.PYTORCH, attn_bias=bias)
    want = orc.hstu_mha_dense(6, 0.5, q, k, v, offs, attn_bias=bias, dtype=torch.float64)
    assert torch.allclose(got, want, atol=1e-12)


def test_hstu_mha_asserts_causal():
    from hstu_amd import hstu_mha

    q = torch.zeros(4, 1, 8)
    with pytest.raises(Exception):
        hstu_mha(4, 0.1, q, q, q, torch.tensor([0, 4]), causal=False)


def test_bench_rejects_multi_gpu():
    r = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stdout


def test_reference_named_ops_registered_with_reference_schemas():
    """generative_recommenders::triton_hstu_attention_{fwd,bwd,delta_bwd}
    exist with the reference's argument names, defaults and mutation sets
    (ops/triton/triton_hstu_attention.py:3166-3185, 3298-3319, 3413-3428)."""
    import hstu_amd  # noqa: F401  (registers the ops)

    ns = torch.ops.generative_recommenders
    fwd = ns.triton_hstu_attention_fwd.default._schema
    assert [a.name for a in fwd.arguments] == [
        "N", "alpha", "q", "k", "v", "seq_offsets", "num_targets", "max_attn_len", "contextual_seq_len",
        "sort_by_length_indices", "enable_tma", "num_softmax_heads", "q_scale", "k_scale", "v_scale"]
    assert [a.default_value for a in fwd.arguments[-3:]] == [1.0, 1.0, 1.0]
    bwd = ns.triton_hstu_attention_bwd.default._schema
    assert [a.name for a in bwd.arguments] == [
        "dout", "q", "k", "v", "dq", "dk", "dv", "seq_offsets", "num_targets", "N", "alpha", "max_attn_len",
        "contextual_seq_len", "sort_by_length_indices", "enable_tma", "num_softmax_heads"]
    assert [a.name for a in bwd.arguments if a.alias_info is not None and a.alias_info.is_write] == ["dq", "dk", "dv"]
    dlt = ns.triton_hstu_attention_delta_bwd.default._schema
    assert [a.name for a in dlt.arguments] == ["dout", "q", "k", "v", "dq", "dk", "dv", "seq_offsets", "N", "alpha",
                                               "k_scale", "v_scale"]
    assert [a.name for a in dlt.arguments if a.alias_info is not None and a.alias_info.is_write] == ["dq", "dk", "dv"]


def test_reference_named_fwd_fake_output_dtype():
    """The fake forward allocates [T, H, Dv] in bf16 for e4m3 inputs, else in
    v's dtype (triton_hstu_attention.py:3508-3524)."""
    import hstu_amd  # noqa: F401
    from torch._subclasses.fake_tensor import FakeTensorMode

    op = torch.ops.generative_recommenders.triton_hstu_attention_fwd
    with FakeTensorMode():
        off = torch.empty(3, dtype=torch.int64)
        q8 = torch.empty(10, 4, 128, dtype=torch.float8_e4m3fn)
        o8 = op(64, 0.1, q8, q8, q8, off, None, 0, 0, None, False, 0)
        q16 = torch.empty(10, 2, 64, dtype=torch.bfloat16)
        v16 = torch.empty(10, 2, 32, dtype=torch.bfloat16)
        o16 = op(64, 0.1, q16, q16, v16, off, None, 0, 0, None, False, 0)
    assert o8.shape == (10, 4, 128) and o8.dtype == torch.bfloat16
    assert o16.shape == (10, 2, 32) and o16.dtype == torch.bfloat16


def test_backward_rejects_mixed_scale_layouts():
    """One scale addressing serves q, k and v in the C ABI, so mixing a scalar
    and per-(token, head) scales is refused before any launch."""
    from hstu_amd import hstu_attention as A

    T, H, D = 8, 2, 128
    q = torch.zeros(T, H, D, dtype=torch.float8_e4m3fn)
    g = [torch.zeros(T, H, D, dtype=torch.bfloat16) for _ in range(3)]
    offs = torch.tensor([0, 8])
    with pytest.raises(ValueError, match="one layout"):
        A._launch_bwd(g[0], q, q, q, *g, offs, None, 16, 0.1, 0, 0, torch.ones(T, H), 1.0, torch.ones(T, H),
                      None, None)


def test_calibrate_scale_buffer_freeze_rule():
    """The scale state [scale, completed, history]: zero while calibrating, then
    max(history) * 1.5 / 448 and frozen (triton_fp8.py:694-749); an all-zero
    value is not a step; a one-element buffer is set from each call."""
    from hstu_amd import fp8 as F

    steps = F.CALIBRATION_STEPS
    buf = torch.zeros(F.fp8_scale_state_size())
    amaxes = [2.0, 0.0, 5.0, 3.0, 1.0, 7.0][: steps + 2]
    got = []
    for a in amaxes:
        got.append(F.calibrate_scale_buffer(buf, torch.full((4, 4), -a)))
    nonzero = [a for a in amaxes if a > 0][:steps]
    want = max(nonzero) * 1.5 / 448
    k = [i for i, a in enumerate(amaxes) if a > 0][steps - 1]
    assert all(v == 0.0 for v in got[:k])
    assert got[k] == pytest.approx(want, rel=1e-6) and all(v == pytest.approx(want, rel=1e-6) for v in got[k:])
    assert float(buf[1]) == steps and F.scale_ready(buf)
    assert float(F.fp8_scale_tensor(buf).reshape(())) == pytest.approx(want, rel=1e-6)
    one = torch.zeros(1)
    assert F.calibrate_scale_buffer(one, torch.full((2,), 3.0), margin=1.0) == pytest.approx(3.0 / 448, rel=1e-6)
    assert F.scale_ready(one) and not F.scale_ready(torch.zeros(F.fp8_scale_state_size()))
    assert F.calibrated_scale(torch.tensor([-4.0, 2.0])).item() == pytest.approx(4.0 * 1.5 / 448, rel=1e-6)


def test_scale_state_known_without_device_reads():
    """A state this module froze is ready without reading it again; a write
    from elsewhere (a checkpoint load) is noticed through the version counter."""
    from hstu_amd import fp8 as F

    buf = torch.zeros(F.fp8_scale_state_size())
    for _ in range(F.CALIBRATION_STEPS):
        F.calibrate_scale_buffer(buf, torch.ones(3))
    v = buf._version
    assert F.scale_ready(buf) and buf._version == v
    buf.zero_()                                   # reset elsewhere
    assert not F.scale_ready(buf)


@pytest.mark.parametrize("bad", [0.0, -1.0, float("inf"), float("nan")])
def test_one_element_scale_needs_finite_positive_value(bad):
    """A one-element scale is usable only once finite and > 0 (the reference's
    activation_scale_value, triton_fp8.py:429-442): a zero buffer runs bf16
    and is calibrated, then ready; the value is read once per version."""
    from hstu_amd import fp8 as F

    s = torch.full((1,), bad)
    assert not F.scale_ready(s)
    F.calibrate_scale_buffer(s, torch.tensor([-2.0, 1.0]))
    assert F.scale_ready(s) and float(s[0]) > 0
    assert F.scale_ready(torch.full((1, 1), 0.25))
    assert not F.scale_ready(torch.zeros(1, 1))


def test_scale_record_is_per_tensor_object():
    """A new tensor on a recycled storage address does not inherit another
    tensor's record: the record holds the tensor as a weak reference."""
    from hstu_amd import fp8 as F

    a = torch.full((1,), 0.5)
    assert F.scale_ready(a)
    F._known[F._key(a)] = (a._version, 1, __import__("weakref").ref(torch.zeros(1)))
    a.zero_()
    assert not F.scale_ready(a)


@pytest.mark.parametrize("amaxes,margin", [([2.0, 3.3, 0.7, 1.1], 1.5), ([1e-3, 7.77, 5.0, 1.0], 1.25),
                                           ([0.123456, 0.2, 0.3, 0.1], 1.5)])
def test_frozen_scale_bits_follow_reference_expression(amaxes, margin):
    """The frozen scale is the reference's fp32 expression
    ``history.amax() * margin / 448`` (triton_fp8.py:737-739) bit for bit,
    and a one-element scale ``amax * margin / 448`` (:724-727)."""
    from hstu_amd import fp8 as F

    buf = torch.zeros(F.fp8_scale_state_size())
    for a in amaxes[: F.CALIBRATION_STEPS]:
        F.calibrate_scale_buffer(buf, torch.tensor([a, -a / 2]), margin=margin)
    hist = torch.tensor(amaxes[: F.CALIBRATION_STEPS], dtype=torch.float32)
    want = hist.amax() * margin / 448.0
    assert torch.equal(buf[0], want)
    one = torch.zeros(1)
    F.calibrate_scale_buffer(one, torch.tensor([amaxes[1]]), margin=margin)
    assert torch.equal(one[0], torch.tensor(amaxes[1], dtype=torch.float32) * margin / 448.0)


def test_uqvk_kernel_reason_and_torch_path():
    """hstu_compute_uqvk(kernel=TRITON) declines what the LayerNorm kernel and
    the bf16 GEMM do not serve (host tensors here) and runs the torch ops,
    equal to the reference's PyTorch composition."""
    import torch.nn.functional as TF

    from hstu_amd import HammerKernel
    from hstu_amd.hstu_preprocess import hstu_compute_uqvk, uqvk_kernel_reason

    g = torch.Generator().manual_seed(0)
    x = torch.randn(5, 512, generator=g)
    nw, nb = torch.randn(512, generator=g), torch.randn(512, generator=g)
    W, b = torch.randn(512, 2048, generator=g) * 0.05, torch.randn(2048, generator=g)
    assert "device" in uqvk_kernel_reason(x, nw, nb, W, b)
    u, q, k, v = hstu_compute_uqvk(x, nw, nb, 1e-6, 4, 128, 128, W, b, kernel=HammerKernel.TRITON)
    uvqk = torch.addmm(b, TF.layer_norm(x, (512,), nw, nb, 1e-6), W)
    assert torch.equal(u, TF.silu(uvqk[:, :512])) and torch.equal(v.reshape(5, 512), uvqk[:, 512:1024])
    assert torch.equal(q.reshape(5, 512), uvqk[:, 1024:1536]) and torch.equal(k.reshape(5, 512), uvqk[:, 1536:])


def test_residual_link_binds_the_preprocess_input():
    """The output block uses a ResidualLink only for the x its preprocess
    forward bound: another tensor, or the same one written in place since,
    gets its residual gradient returned the ordinary way."""
    from hstu_amd.hstu_linear import ResidualLink

    x = torch.zeros(4, 8)
    link = ResidualLink()
    assert not link.bound_to(x)
    link.bind(x)
    assert link.bound_to(x) and not link.bound_to(x.clone()) and not link.bound_to(x.view(8, 4))
    x.add_(1.0)
    assert not link.bound_to(x)
    link.grad = torch.ones(1)
    assert link.take() is not None and link.take() is None
