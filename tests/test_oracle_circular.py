"""CPU pinning of the circular FFT-conv oracle (no GPU).

The FFT restatement (``circular_fftconv_torch``) is checked against the
float64 brute force (``circular_conv_direct_np``), and the brute force against
facts that fix it independently: a delta at the centre tap is the identity, a
delta at tap ``j`` is a roll by ``j - (K-1)//2``, the reference test's own
spatial formula (circular padding ``K//2`` left / ``K-1-K//2`` right, flipped
kernel, grouped conv; tests/ops/test_circular_fftconv.py:69-105) written with
``torch.nn.functional``, and separability of a rank-one kernel.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as Fn

from oracle.circular_ref import circular_conv_direct_np, circular_fftconv_torch
from oracle.fftconv_ref import rel_l2


CASES = [((2, 3, 16), (1, 3, 5)), ((2, 3, 16), (2, 3, 16)), ((1, 2, 12), (1, 2, 1)), ((1, 2, 9), (1, 2, 4)),
         ((2, 2, 8, 12), (1, 2, 3, 6)), ((1, 3, 16, 16), (1, 3, 16, 16)), ((2, 2, 6, 5), (2, 2, 6, 2)),
         ((1, 2, 4, 6, 8), (1, 2, 3, 4, 5)), ((2, 1, 8, 8, 8), (2, 1, 8, 1, 7))]


def _spatial_reference(x, k):
    """Circular pad K//2 / K-1-K//2 per axis, flip the kernel, grouped conv (float64)."""
    nd = x.dim() - 2
    K = k.shape[2:]
    pad = []
    for d in reversed(range(nd)):
        pad += [K[d] // 2, K[d] - 1 - K[d] // 2]
    xp = Fn.pad(x, pad, mode="circular")
    w = torch.flip(k, dims=tuple(range(2, 2 + nd)))
    conv = (Fn.conv1d, Fn.conv2d, Fn.conv3d)[nd - 1]
    if k.shape[0] == 1:
        return conv(xp, w[0].unsqueeze(1), groups=x.shape[1])
    return torch.stack([conv(xp[b:b + 1], w[b].unsqueeze(1), groups=x.shape[1])[0] for b in range(x.shape[0])])


@pytest.mark.parametrize("xs,ks", CASES)
def test_fft_restatement_matches_brute_force(xs, ks):
    rng = np.random.default_rng(sum(xs) + sum(ks))
    x = rng.standard_normal(xs)
    k = rng.standard_normal(ks)
    s = rng.standard_normal(xs[1])
    ref = circular_conv_direct_np(x, k, s)
    yt = circular_fftconv_torch(torch.tensor(x, dtype=torch.float32), torch.tensor(k, dtype=torch.float32),
                                torch.tensor(s, dtype=torch.float32))
    assert rel_l2(ref, yt) < 1e-5


@pytest.mark.parametrize("xs,ks", CASES)
def test_brute_force_matches_spatial_padding_formula(xs, ks):
    rng = np.random.default_rng(7 + sum(xs))
    x = rng.standard_normal(xs)
    k = rng.standard_normal(ks)
    ref = _spatial_reference(torch.tensor(x), torch.tensor(k)).numpy()
    assert rel_l2(ref, circular_conv_direct_np(x, k)) < 1e-13


def test_centre_delta_is_identity_and_offset_delta_is_roll():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((1, 2, 10, 8))
    K = (6, 5)
    c = ((K[0] - 1) // 2, (K[1] - 1) // 2)
    k = np.zeros((1, 2) + K)
    k[:, :, c[0], c[1]] = 1.0
    np.testing.assert_allclose(circular_conv_direct_np(x, k), x, atol=1e-14)
    k = np.zeros((1, 2) + K)
    k[:, :, 4, 0] = 1.0  # y[n] = x[n + c - j]  ->  roll by j - c
    np.testing.assert_allclose(circular_conv_direct_np(x, k), np.roll(x, (4 - c[0], 0 - c[1]), axis=(2, 3)), atol=1e-14)
    yt = circular_fftconv_torch(torch.tensor(x, dtype=torch.float32), torch.tensor(k, dtype=torch.float32))
    np.testing.assert_allclose(yt.numpy(), np.roll(x, (4 - c[0], -c[1]), axis=(2, 3)), atol=1e-5)


def test_rank_one_kernel_is_separable():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((1, 1, 12, 10))
    a, b = rng.standard_normal(5), rng.standard_normal(4)
    k2 = np.outer(a, b)[None, None]
    t = circular_conv_direct_np(np.transpose(x, (0, 3, 1, 2)).reshape(1, 10, 12), np.tile(a, (1, 10, 1)))
    t = np.transpose(t.reshape(1, 10, 1, 12), (0, 2, 3, 1))
    t = circular_conv_direct_np(t.reshape(1, 12, 10), np.tile(b, (1, 12, 1))).reshape(1, 1, 12, 10)
    assert rel_l2(t, circular_conv_direct_np(x, k2)) < 1e-13


def test_gradients_are_adjoint_convolution():
    """d<y, g>/dx is the circular correlation with the same kernel; d/dk is the lagged cross-correlation."""
    rng = np.random.default_rng(3)
    x = torch.tensor(rng.standard_normal((2, 2, 8, 6)), requires_grad=True)
    k = torch.tensor(rng.standard_normal((1, 2, 5, 4)), requires_grad=True)
    g = rng.standard_normal((2, 2, 8, 6))
    y = circular_fftconv_torch(x.float(), k.float())
    (y.double() * torch.tensor(g)).sum().backward()
    c = (2, 1)
    xn, kn = x.detach().numpy(), k.detach().numpy()
    gx = np.zeros_like(xn)
    gk = np.zeros_like(kn)
    for j0 in range(5):
        for j1 in range(4):
            # y[n] += k[j] x[n + c - j]  =>  gx[m] += k[j] g[m - c + j], gk[j] = sum_n g[n] x[n + c - j]
            gx += kn[:, :, j0, j1][..., None, None] * np.roll(g, (c[0] - j0, c[1] - j1), axis=(2, 3))
            gk[0, :, j0, j1] = (g * np.roll(xn, (j0 - c[0], j1 - c[1]), axis=(2, 3))).sum(axis=(0, 2, 3))
    assert rel_l2(gx, x.grad.numpy()) < 1e-5
    assert rel_l2(gk, k.grad.numpy()) < 1e-5


# --- mixed boundary conditions (ops/mixed_fftconv.py) -----------------------
from oracle.circular_ref import mixed_conv_direct_np, mixed_fftconv_torch  # noqa: E402
from oracle.fftconv_ref import fftconv_nd_np  # noqa: E402

MIXED = [((2, 2, 16, 12), (1, 2, 5, 7), (True, False)), ((1, 3, 10, 16), (1, 3, 20, 3), (False, True)),
         ((2, 2, 8, 6, 16), (2, 2, 3, 5, 4), (True, True, False)), ((1, 1, 6, 8, 5), (1, 1, 4, 8, 9), (False, True, False)),
         ((1, 2, 12, 9), (1, 2, 4, 18), (True, False))]


@pytest.mark.parametrize("xs,ks,per", MIXED)
def test_mixed_restatement_matches_brute_force(xs, ks, per):
    rng = np.random.default_rng(sum(xs) + 3 * sum(ks))
    x = rng.standard_normal(xs)
    k = rng.standard_normal(ks)
    s = rng.standard_normal(xs[1])
    ref = mixed_conv_direct_np(x, k, per, s)
    yt = mixed_fftconv_torch(torch.tensor(x, dtype=torch.float32), torch.tensor(k, dtype=torch.float32), per,
                             torch.tensor(s, dtype=torch.float32))
    assert rel_l2(ref, yt) < 1e-5


@pytest.mark.parametrize("L,K", [(16, 5), (16, 6), (9, 18), (7, 1), (1, 2), (33, 20)])
def test_mixed_1d_zero_padded_is_numpy_full_convolution_cropped(L, K):
    """1D periodic=(False,) ("same", ops/fftconv.py:603-660): numpy's full linear convolution sliced at
    [K//2, K//2 + L) (not numpy's own mode="same", which crops at (K-1)//2); the FFT restatement agrees."""
    rng = np.random.default_rng(L * 31 + K)
    x = rng.standard_normal((2, 3, L))
    k = rng.standard_normal((1, 3, K))
    s = rng.standard_normal(3)
    ref = np.stack([[np.convolve(x[b, h], k[0, h])[K // 2:K // 2 + L] + s[h] * x[b, h] for h in range(3)]
                    for b in range(2)])
    assert rel_l2(ref, mixed_conv_direct_np(x, k, (False,), s)) < 1e-13
    yt = mixed_fftconv_torch(torch.tensor(x), torch.tensor(k), (False,), torch.tensor(s), compute_dtype=torch.float64)
    assert rel_l2(ref, yt) < 1e-12
    # periodic=(True,) (K <= L) is the circular wrap of the same sum
    if K <= L:
        c = (K - 1) // 2
        refc = np.stack([[sum(k[0, h, j] * np.roll(x[b, h], j - c) for j in range(K)) for h in range(3)]
                         for b in range(2)])
        assert rel_l2(refc, mixed_conv_direct_np(x, k, (True,))) < 1e-13


@pytest.mark.parametrize("xs,ks", [((2, 2, 9, 7), (1, 2, 5, 3)), ((1, 2, 5, 6, 4), (1, 2, 3, 4, 8))])
def test_mixed_brute_force_uniform_cases(xs, ks):
    """All periodic = the circular brute force; all zero = the zero-padded "same" restatement."""
    rng = np.random.default_rng(11)
    x = rng.standard_normal(xs)
    k = rng.standard_normal(ks)
    nd = len(xs) - 2
    assert rel_l2(circular_conv_direct_np(x, k), mixed_conv_direct_np(x, k, (True,) * nd)) < 1e-14
    assert rel_l2(fftconv_nd_np(x, k[0]), mixed_conv_direct_np(x, k, (False,) * nd)) < 1e-12


def test_float32_ramp_error_grows_with_kernel_length():
    """The reference computes its ramp angles 2*pi*c*f in float32 (circular_fftconv.py:_PhaseRampCache1D.get);
    at K = L = 4096 the angles reach ~pi*2047 and their rounding costs ~1e-4 relative, while the float64
    restatement matches the brute force.  The GPU parity tests therefore compare against float64."""
    rng = np.random.default_rng(12)
    x = rng.standard_normal((1, 2, 4096))
    k = rng.standard_normal((1, 2, 4096))
    ref = circular_conv_direct_np(x, k)
    y64 = circular_fftconv_torch(torch.tensor(x), torch.tensor(k), compute_dtype=torch.float64)
    y32 = circular_fftconv_torch(torch.tensor(x, dtype=torch.float32), torch.tensor(k, dtype=torch.float32))
    assert rel_l2(ref, y64) < 1e-12
    assert rel_l2(ref, y32) > 3e-5
    # short kernels keep the float32 angles small: the reference arithmetic is then accurate
    k7 = k[..., :7]
    y32s = circular_fftconv_torch(torch.tensor(x, dtype=torch.float32), torch.tensor(k7, dtype=torch.float32))
    assert rel_l2(circular_conv_direct_np(x, k7), y32s) < 2e-6
