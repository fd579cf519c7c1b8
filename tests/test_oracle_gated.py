"""CPU pinning of the gated restatement (no GPU): identity gates with unit values reduce it to the pinned causal
conv of q * k; the sigmoid / silu gates are torch's own (silu(x) = x sigmoid(x) checked); and its autograd
gradients match the chain rule written out with the causal conv's adjoint (oracle.direct, float64)."""

import numpy as np
import torch

from oracle import direct
from oracle.fftconv_ref import causal_fftconv1d_torch, rel_l2
from oracle.gated_ref import gated_causal_fftconv1d_torch


def test_identity_gates_reduce_to_conv_of_product():
    torch.manual_seed(0)
    q, k = torch.randn(2, 3, 40), torch.randn(2, 3, 40)
    w = torch.randn(1, 3, 9)
    s = torch.randn(3)
    y = gated_causal_fftconv1d_torch(q, k, torch.ones(2, 3, 40), w, s, "identity")
    assert torch.equal(y, causal_fftconv1d_torch(q * k, w, s))


def test_silu_is_x_sigmoid_x():
    x = torch.linspace(-6, 6, 101, dtype=torch.float64)
    assert torch.allclose(torch.nn.functional.silu(x), x * torch.sigmoid(x))


def test_gradients_match_written_out_chain_rule():
    rng = np.random.default_rng(1)
    B, H, L, K = 2, 3, 30, 7
    q, k, v, g = (rng.standard_normal((B, H, L)) for _ in range(4))
    w = rng.standard_normal((H, K))
    s = rng.standard_normal(H)
    qt, kt, vt = (torch.tensor(a, requires_grad=True) for a in (q, k, v))
    wt, st = torch.tensor(w[None], requires_grad=True), torch.tensor(s, requires_grad=True)
    y = gated_causal_fftconv1d_torch(qt, kt, vt, wt, st, "silu", "sigmoid")
    y.backward(torch.tensor(g))
    sig = lambda a: 1 / (1 + np.exp(-a))  # noqa: E731
    z = q * k * sig(k)
    y1 = direct.causal_conv1d(z, w) + s[None, :, None] * z
    dy1 = g * sig(v)
    dv = g * y1 * sig(v) * (1 - sig(v))
    dz_conv, dw = direct.causal_conv1d_bwd(dy1, z, w)
    dz = dz_conv + s[None, :, None] * dy1
    dq = dz * k * sig(k)
    dk = dz * q * sig(k) * (1 + k * (1 - sig(k)))
    assert rel_l2(dq, qt.grad) < 1e-5 and rel_l2(dk, kt.grad) < 1e-5 and rel_l2(dv, vt.grad) < 1e-5
    assert rel_l2(dw, wt.grad[0]) < 1e-5
    assert rel_l2((dy1 * z).sum(axis=(0, 2)), st.grad) < 1e-5


def test_nd_gates_around_a_centre_delta_filter():
    """A centre delta (index K//2 on zero-padded axes, (K-1)//2 on periodic ones) makes the conv the identity, so
    the gated op is (z + s z) * act2(v) with z = q * act1(k) -- a closed form independent of the FFT recipe."""
    from oracle.gated_ref import gated_fftconv_nd_torch

    torch.manual_seed(2)
    for periodic, ks in (((False, False), (5, 4)), ((True, False, True), (3, 4, 5))):
        S = (8, 6) if len(ks) == 2 else (8, 6, 8)
        q, kg, v = (torch.randn(2, 3, *S, dtype=torch.float64) for _ in range(3))
        s = torch.randn(3, dtype=torch.float64)
        kernel = torch.zeros(1, 3, *ks, dtype=torch.float64)
        centre = tuple((kd - 1) // 2 if p else kd // 2 for kd, p in zip(ks, periodic))
        kernel[(0, slice(None)) + centre] = 1.0
        y = gated_fftconv_nd_torch(q, kg, v, kernel, periodic, s, gate="sigmoid", gate_2="silu",
                                   compute_dtype=torch.float64)
        z = q * torch.sigmoid(kg)
        ref = (z + s.view(1, 3, *([1] * len(S))) * z) * torch.nn.functional.silu(v)
        assert torch.allclose(y, ref, atol=1e-12)
