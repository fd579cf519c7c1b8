"""CPU pinning of the channel-RMSNorm restatement (oracle/norm_ref.py): closed-form normalised values, scale
invariance, finite-difference gradients in float64, orthogonality of the input gradient to u at eps = 0, the gate
as torch's own sigmoid / silu, and the channels-first layout as the channels-last one moved back."""

import math

import pytest
import torch

from oracle.norm_ref import gated_channel_groupnorm_ref, gated_channel_layernorm_ref, gated_channel_rmsnorm_ref, l2norm_ref


def test_closed_form_ramp():
    # u_c = a (c + 1) at every position: mean_c u^2 = a^2 (C + 1)(2C + 1) / 6
    B, C, S, a, eps = 2, 7, 5, 0.37, 1e-3
    ramp = torch.arange(1, C + 1, dtype=torch.float64)
    y = (a * ramp).view(1, C, 1).expand(B, C, S).contiguous()
    w = torch.linspace(0.5, 2.0, C, dtype=torch.float64)
    out = gated_channel_rmsnorm_ref(y, None, w, eps)
    ms = a * a * (C + 1) * (2 * C + 1) / 6
    want = w * (a * ramp) / math.sqrt(ms + eps)
    assert out.shape == (B, S, C)
    assert torch.allclose(out, want.view(1, 1, C).expand(B, S, C), rtol=1e-12, atol=0)


def test_scale_invariance_and_unit_rms():
    torch.manual_seed(0)
    y = torch.randn(3, 16, 4, 5, dtype=torch.float64)
    w = torch.ones(16, dtype=torch.float64)
    o1 = gated_channel_rmsnorm_ref(y, None, w, 0.0)
    o2 = gated_channel_rmsnorm_ref(7.5 * y, None, w, 0.0)
    assert torch.allclose(o1, o2, rtol=1e-12, atol=1e-12)
    assert torch.allclose(o1.pow(2).mean(-1), torch.ones(3, 4, 5, dtype=torch.float64), rtol=1e-12)


def test_gate_and_layouts():
    torch.manual_seed(1)
    y, v = torch.randn(2, 6, 9, dtype=torch.float64), torch.randn(2, 6, 9, dtype=torch.float64)
    w = torch.randn(6, dtype=torch.float64)
    for act, f in ((1, torch.sigmoid), (2, lambda t: t * torch.sigmoid(t)), (0, lambda t: t)):
        last = gated_channel_rmsnorm_ref(y, v, w, 1e-6, act, channels_last=True)
        assert torch.allclose(last, gated_channel_rmsnorm_ref(y * f(v), None, w, 1e-6), rtol=1e-13, atol=0)
        first = gated_channel_rmsnorm_ref(y, v, w, 1e-6, act, channels_last=False)
        assert torch.equal(first, last.movedim(-1, 1))


def test_gradcheck_float64():
    torch.manual_seed(2)
    y = torch.randn(2, 5, 3, dtype=torch.float64, requires_grad=True)
    v = torch.randn(2, 5, 3, dtype=torch.float64, requires_grad=True)
    w = torch.randn(5, dtype=torch.float64, requires_grad=True)
    for act in (0, 1, 2):
        assert torch.autograd.gradcheck(lambda a, b, c: gated_channel_rmsnorm_ref(a, b, c, 1e-3, act), (y, v, w))


def test_input_gradient_orthogonal_to_u_at_zero_eps():
    # out is invariant to scaling u, so d/dlambda out(lambda u) = 0  =>  sum_c du_c u_c = 0 per position
    torch.manual_seed(3)
    u = torch.randn(2, 8, 11, dtype=torch.float64, requires_grad=True)
    w = torch.randn(8, dtype=torch.float64)
    out = gated_channel_rmsnorm_ref(u, None, w, 0.0)
    (du,) = torch.autograd.grad(out, u, torch.randn_like(out))
    assert (du * u).sum(1).abs().max() < 1e-12


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32, torch.bfloat16, torch.float16])
def test_l2norm_restatement_matches_torch_normalize(dtype):
    """The QK-norm restatement equals torch's F.normalize (the reference's L2Norm body) on every dtype."""
    torch.manual_seed(0)
    x = (torch.randn(3, 40, 7, 5) * 3).to(dtype)
    for dim in (1, -1):
        assert torch.equal(l2norm_ref(x, dim), torch.nn.functional.normalize(x, p=2.0, dim=dim))


def test_l2norm_closed_forms_and_clamp():
    x = torch.tensor([[[3.0], [4.0]]], dtype=torch.float64)   # [B=1, C=2, S=1]
    assert torch.allclose(l2norm_ref(x), torch.tensor([[[0.6], [0.8]]], dtype=torch.float64), rtol=0, atol=1e-15)
    tiny = torch.full((1, 4, 1), 1e-5, dtype=torch.float64)   # ||x|| = 2e-5 < eps = 1e-3: x / eps
    assert torch.allclose(l2norm_ref(tiny, eps=1e-3), tiny / 1e-3, rtol=1e-15, atol=0)
    y = torch.randn(2, 9, 6, dtype=torch.float64)
    assert torch.allclose(torch.linalg.vector_norm(l2norm_ref(y), dim=1), torch.ones(2, 6, dtype=torch.float64))
    assert torch.allclose(l2norm_ref(5.0 * y), l2norm_ref(y), rtol=1e-14, atol=1e-14)


def test_l2norm_gradcheck_float64():
    y = torch.randn(2, 5, 3, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(lambda t: l2norm_ref(t, 1, 1e-12), (y,))
    small = (torch.randn(1, 3, 2, dtype=torch.float64) * 1e-4).requires_grad_(True)  # clamped branch
    assert torch.autograd.gradcheck(lambda t: l2norm_ref(t, 1, 1e-2), (small,))


# LayerNorm over channels (the pixelhyena_norm site with torch.nn.LayerNorm(C))

@pytest.mark.parametrize("affine", [True, False])
def test_layernorm_restatement_matches_torch_layer_norm_float64(affine):
    torch.manual_seed(3)
    y = torch.randn(2, 12, 5, 3, dtype=torch.float64)
    v = torch.randn(2, 12, 5, 3, dtype=torch.float64)
    w = torch.randn(12, dtype=torch.float64) if affine else None
    b = torch.randn(12, dtype=torch.float64) if affine else None
    for act, f in ((0, lambda t: t), (1, torch.sigmoid), (2, torch.nn.functional.silu)):
        got = gated_channel_layernorm_ref(y, v, w, b, 1e-5, act, channels_last=True)
        want = torch.nn.functional.layer_norm((y * f(v)).movedim(1, -1), (12,), w, b, 1e-5)
        assert torch.allclose(got, want, rtol=1e-12, atol=1e-12)
    cf = gated_channel_layernorm_ref(y, None, w, b, 1e-5, 0, channels_last=False)
    assert torch.allclose(cf, torch.nn.functional.layer_norm(y.movedim(1, -1), (12,), w, b, 1e-5).movedim(-1, 1),
                          rtol=1e-12, atol=1e-12)


def test_layernorm_closed_form_and_invariances():
    y = torch.tensor([1.0, 2.0, 3.0], dtype=torch.float64).view(1, 3, 1)
    out = gated_channel_layernorm_ref(y, None, None, None, 0.0, 0)
    r = math.sqrt(1.5)
    assert torch.allclose(out.view(3), torch.tensor([-r, 0.0, r], dtype=torch.float64), rtol=1e-14, atol=1e-14)
    torch.manual_seed(4)
    z = torch.randn(2, 9, 7, dtype=torch.float64)
    o1 = gated_channel_layernorm_ref(z, None, None, None, 0.0, 0)
    o2 = gated_channel_layernorm_ref(3.5 * z + 11.0, None, None, None, 0.0, 0)  # shift and scale invariant
    assert torch.allclose(o1, o2, rtol=1e-11, atol=1e-11)
    assert torch.allclose(o1.mean(1), torch.zeros(2, 7, dtype=torch.float64), atol=1e-13)
    assert torch.allclose(o1.pow(2).mean(1), torch.ones(2, 7, dtype=torch.float64), rtol=1e-12)


def test_layernorm_gradcheck_float64():
    torch.manual_seed(5)
    y = torch.randn(2, 6, 4, dtype=torch.float64, requires_grad=True)
    v = torch.randn(2, 6, 4, dtype=torch.float64, requires_grad=True)
    w = torch.randn(6, dtype=torch.float64, requires_grad=True)
    b = torch.randn(6, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(lambda *t: gated_channel_layernorm_ref(*t, 1e-3, 2, True), (y, v, w, b))


# GroupNorm over channels, channels-first (the pixelhyena_norm site with torch.nn.GroupNorm(G, C))

@pytest.mark.parametrize("groups", [1, 3, 12])
@pytest.mark.parametrize("affine", [True, False])
def test_groupnorm_restatement_matches_torch_group_norm_float64(groups, affine):
    torch.manual_seed(6)
    y = torch.randn(2, 12, 5, 3, dtype=torch.float64)
    v = torch.randn(2, 12, 5, 3, dtype=torch.float64)
    w = torch.randn(12, dtype=torch.float64) if affine else None
    b = torch.randn(12, dtype=torch.float64) if affine else None
    for act, f in ((0, lambda t: t), (1, torch.sigmoid), (2, torch.nn.functional.silu)):
        got = gated_channel_groupnorm_ref(y, v, w, b, groups, 1e-5, act)
        want = torch.nn.functional.group_norm(y * f(v), groups, w, b, 1e-5)
        assert torch.allclose(got, want, rtol=1e-12, atol=1e-12)


def test_groupnorm_one_group_per_channel_is_instance_norm():
    torch.manual_seed(7)
    y = torch.randn(3, 8, 4, 5, dtype=torch.float64)
    w = torch.randn(8, dtype=torch.float64)
    b = torch.randn(8, dtype=torch.float64)
    got = gated_channel_groupnorm_ref(y, None, w, b, 8, 1e-5, 0)
    want = torch.nn.functional.instance_norm(y, weight=w, bias=b, eps=1e-5)
    assert torch.allclose(got, want, rtol=1e-12, atol=1e-12)


def test_groupnorm_closed_form_one_group():
    # one group over C = 2 channels x S = 2 positions: values 1, 2, 3, 4 -> mean 2.5, var 1.25
    y = torch.tensor([[[1.0, 2.0], [3.0, 4.0]]], dtype=torch.float64)
    out = gated_channel_groupnorm_ref(y, None, None, None, 1, 0.0, 0)
    r = 1.0 / math.sqrt(1.25)
    want = torch.tensor([[[-1.5 * r, -0.5 * r], [0.5 * r, 1.5 * r]]], dtype=torch.float64)
    assert torch.allclose(out, want, rtol=1e-14, atol=1e-14)
    # w, b per channel after the group statistics: channel 1 scaled by 2 and shifted by 1
    o2 = gated_channel_groupnorm_ref(y, None, torch.tensor([1.0, 2.0], dtype=torch.float64),
                                     torch.tensor([0.0, 1.0], dtype=torch.float64), 1, 0.0, 0)
    assert torch.allclose(o2[0, 1], 2.0 * want[0, 1] + 1.0, rtol=1e-14, atol=1e-14)
    assert torch.allclose(o2[0, 0], want[0, 0], rtol=1e-14, atol=1e-14)


def test_groupnorm_float32_rounding_once():
    # a 16-bit input: the statistics in float64, the affine in float32, one rounding to the input dtype
    torch.manual_seed(8)
    y = torch.randn(2, 6, 33).to(torch.bfloat16)
    w, b = torch.randn(6), torch.randn(6)
    got = gated_channel_groupnorm_ref(y, None, w, b, 2, 1e-5, 0)
    assert got.dtype == torch.bfloat16
    want = torch.nn.functional.group_norm(y.double(), 2, w.double(), b.double(), 1e-5)
    assert (got.double() - want).abs().max() <= 2 ** -7 * want.abs().max()


def test_groupnorm_gradcheck_float64():
    torch.manual_seed(9)
    y = torch.randn(2, 6, 4, dtype=torch.float64, requires_grad=True)
    v = torch.randn(2, 6, 4, dtype=torch.float64, requires_grad=True)
    w = torch.randn(6, dtype=torch.float64, requires_grad=True)
    b = torch.randn(6, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(lambda *t: gated_channel_groupnorm_ref(*t, 3, 1e-3, 2), (y, v, w, b))
