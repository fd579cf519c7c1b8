"""CPU tests pinning the oracle (no GPU).

The FFT restatements in oracle/fftconv_ref.py are checked against:
  * brute-force float64 direct convolutions (oracle/direct_conv.c, no FFT),
  * the committed golden fixtures tests/golden/causal1d.npz (written by the
    same brute force; checked here so a regenerated fixture cannot drift),
  * closed forms: delta filter, shifted delta, causality, linearity, the
    wrap-around of the reference FFT length when K > L+1,
  * torch autograd of the restatement == the float64 adjoint.
"""

import os

import numpy as np
import pytest
import torch

from oracle import direct
from oracle.fftconv_ref import (
    causal_fftconv1d_bwd_np,
    causal_fftconv1d_chunked_torch,
    causal_fftconv1d_np,
    causal_fftconv1d_torch,
    rel_l2,
    round_bf16_np,
)


GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "causal1d.npz")

SHAPES = [(2, 4, 64, 7), (1, 3, 32, 32), (2, 2, 16, 3), (1, 2, 17, 5), (1, 2, 16, 24), (1, 2, 9, 18), (2, 3, 33, 34)]


def _case(B, H, L, K, seed=0):
    rng = np.random.default_rng(seed)
    return (
        rng.standard_normal((B, H, L)),
        rng.standard_normal((H, K)),
        rng.standard_normal(H),
        rng.standard_normal((B, H, L)),
    )


@pytest.mark.parametrize("B,H,L,K", SHAPES)
def test_np_restatement_matches_brute_force(B, H, L, K):
    x, k, s, _ = _case(B, H, L, K)
    y_bf = direct.causal_conv1d(x, k) + s[None, :, None] * x
    y_np = causal_fftconv1d_np(x, k, s)
    assert rel_l2(y_bf, y_np) < 1e-12


@pytest.mark.parametrize("B,H,L,K", SHAPES)
def test_torch_restatement_matches_brute_force(B, H, L, K):
    x, k, s, _ = _case(B, H, L, K, seed=1)
    y_bf = direct.causal_conv1d(x, k) + s[None, :, None] * x
    y_t = causal_fftconv1d_torch(torch.tensor(x, dtype=torch.float32), torch.tensor(k, dtype=torch.float32)[None],
                                 torch.tensor(s, dtype=torch.float32))
    assert rel_l2(y_bf, y_t) < 1e-5


@pytest.mark.parametrize("B,H,L,K", SHAPES)
def test_bwd_np_matches_brute_force_adjoint(B, H, L, K):
    x, k, s, g = _case(B, H, L, K, seed=2)
    gx_bf, gk_bf = direct.causal_conv1d_bwd(g, x, k)
    gx, gk, gs = causal_fftconv1d_bwd_np(g, x, k, True, s)
    assert rel_l2(gx_bf + s[None, :, None] * g, gx) < 1e-12
    assert rel_l2(gk_bf, gk) < 1e-12
    assert rel_l2((g * x).sum(axis=(0, 2)), gs) < 1e-12


@pytest.mark.parametrize("B,H,L,K", SHAPES)
def test_torch_autograd_matches_adjoint(B, H, L, K):
    x, k, s, g = _case(B, H, L, K, seed=3)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    kt = torch.tensor(k, dtype=torch.float64, requires_grad=True)
    st = torch.tensor(s, dtype=torch.float64, requires_grad=True)
    y = causal_fftconv1d_torch(xt, kt[None], st)
    # the restatement computes in fp32 internally; compare with a loose bound
    y.backward(torch.tensor(g, dtype=torch.float64))
    gx, gk, gs = causal_fftconv1d_bwd_np(g, x, k, True, s)
    assert rel_l2(gx, xt.grad) < 1e-5
    assert rel_l2(gk, kt.grad) < 1e-5
    assert rel_l2(gs, st.grad) < 1e-5


def test_golden_fixtures_match_brute_force_and_restatements():
    d = np.load(GOLDEN)
    n = int(d["n_causal"])
    assert n >= 5
    for i in range(n):
        B, H, L, K = (int(v) for v in d[f"c{i}_shape"])
        x, k, s, g = d[f"c{i}_x"], d[f"c{i}_k"], d[f"c{i}_s"], d[f"c{i}_g"]
        # the fixture itself equals the brute force (detects a stale fixture)
        assert rel_l2(direct.causal_conv1d(x, k) + s[None, :, None] * x, d[f"c{i}_y"]) < 1e-13
        assert rel_l2(d[f"c{i}_y"], causal_fftconv1d_np(x, k, s)) < 1e-12
        gx, gk, gs = causal_fftconv1d_bwd_np(g, x, k, True, s)
        assert rel_l2(d[f"c{i}_gx"], gx) < 1e-12
        assert rel_l2(d[f"c{i}_gk"], gk) < 1e-12
        assert rel_l2(d[f"c{i}_gs"], gs) < 1e-12


def test_delta_filter_is_identity_plus_shortcut():
    x, _, s, _ = _case(2, 3, 50, 1, seed=4)
    k = np.zeros((3, 50))
    k[:, 0] = 1.0
    y = causal_fftconv1d_np(x, k, s)
    np.testing.assert_allclose(y, (1 + s[None, :, None]) * x, atol=1e-12)


@pytest.mark.parametrize("j", [1, 5, 49])
def test_shifted_delta_is_causal_shift(j):
    x, _, _, _ = _case(1, 2, 50, 1, seed=5)
    k = np.zeros((2, 50))
    k[:, j] = 1.0
    y = causal_fftconv1d_np(x, k)
    ref = np.zeros_like(x)
    ref[..., j:] = x[..., :-j]
    np.testing.assert_allclose(y, ref, atol=1e-12)


def test_wraparound_when_kernel_longer_than_l_plus_one():
    # K = L + 3 > L + 1: F = 2L and tap m = 2L - 1 + ... wraps onto early outputs.
    L = 8
    x = np.zeros((1, 1, L))
    x[0, 0, 0] = 1.0
    k = np.zeros((1, L + 3))
    k[0, L + 2] = 1.0  # contributes to full[L+2] only: folds onto index L+2-2L < 0 -> none
    assert np.abs(causal_fftconv1d_np(x, k)).max() < 1e-12
    x2 = np.zeros((1, 1, L))
    x2[0, 0, L - 1] = 1.0  # full[L-1 + L+2] = full[2L+1] -> folds to y[1]
    y = causal_fftconv1d_np(x2, k)
    expect = np.zeros((1, 1, L))
    expect[0, 0, 1] = 1.0
    np.testing.assert_allclose(y, expect, atol=1e-12)
    np.testing.assert_allclose(direct.causal_conv1d(x2, k), expect, atol=1e-12)


def test_causality_by_perturbation():
    x, k, _, _ = _case(1, 2, 40, 40, seed=6)
    y0 = causal_fftconv1d_np(x, k)
    x2 = x.copy()
    x2[..., 25] += 3.0
    y1 = causal_fftconv1d_np(x2, k)
    np.testing.assert_allclose(y0[..., :25], y1[..., :25], atol=1e-12)
    assert np.abs(y0[..., 25:] - y1[..., 25:]).max() > 1e-3


def test_linearity():
    x, k, _, g = _case(2, 2, 30, 11, seed=7)
    a = 0.37
    lhs = causal_fftconv1d_np(a * x + g, k)
    rhs = a * causal_fftconv1d_np(x, k) + causal_fftconv1d_np(g, k)
    np.testing.assert_allclose(lhs, rhs, atol=1e-12)


def test_chunked_equals_unchunked():
    # CPU torch.fft vectorises across the batch, so only per-element rounding
    # may differ between chunkings (the HIP path is bitwise; see GPU tests).
    x, k, s, _ = _case(2, 10, 64, 9, seed=8)
    xt, kt, st = (torch.tensor(v, dtype=torch.float32) for v in (x, k, s))
    y = causal_fftconv1d_torch(xt, kt[None], st)
    yc = causal_fftconv1d_chunked_torch(xt, kt[None], st, chunk_size=3)
    torch.testing.assert_close(y, yc, rtol=1e-6, atol=1e-6)


def test_bf16_rounding_helper_matches_torch():
    rng = np.random.default_rng(9)
    a = (rng.standard_normal(10000) * 10.0 ** rng.integers(-5, 5, 10000)).astype(np.float32)
    a[:4] = [0.0, -0.0, np.inf, -np.inf]
    ref = torch.tensor(a).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(round_bf16_np(a), ref)


def test_bf16_output_cast_and_shortcut_rounding():
    # bf16 path of the restatement: cast of the conv, then bf16 product and sum.
    x, k, s, _ = _case(1, 2, 32, 5, seed=10)
    xb = torch.tensor(x, dtype=torch.float32).to(torch.bfloat16)
    kt = torch.tensor(k, dtype=torch.float32)[None]
    sb = torch.tensor(s, dtype=torch.float32).to(torch.bfloat16)
    y = causal_fftconv1d_torch(xb, kt, sb)
    assert y.dtype == torch.bfloat16
    conv = causal_fftconv1d_np(xb.float().numpy(), k)
    sx = round_bf16_np(sb.float().numpy()[None, :, None] * xb.float().numpy())
    expect = round_bf16_np(round_bf16_np(conv) + sx)
    # fp32 FFT vs fp64 conv may flip a bf16 rounding: allow a 1-ulp difference
    diff = np.abs(y.float().numpy() - expect)
    assert (diff <= np.abs(expect) * 2 ** -7 + 1e-30).all()


@pytest.mark.parametrize("B,H,L,K", [(3, 4, 64, 17), (2, 3, 50, 100), (2, 2, 33, 33)])
def test_per_sample_filters_match_brute_force_per_image(B, H, L, K):
    """Kernel [B, H, K] (fftconv.py:571-574 allows a leading batch): image b uses filter b -- the brute force
    run image by image, and the autograd gradients are each image's own adjoint (gk per image, not summed)."""
    rng = np.random.default_rng(B * 7 + K)
    x = rng.standard_normal((B, H, L))
    k = rng.standard_normal((B, H, K))
    g = rng.standard_normal((B, H, L))
    xt = torch.tensor(x, requires_grad=True)
    kt = torch.tensor(k, requires_grad=True)
    y = causal_fftconv1d_torch(xt, kt)
    y.backward(torch.tensor(g))
    for b in range(B):
        assert rel_l2(direct.causal_conv1d(x[b:b + 1], k[b]), y[b:b + 1].detach()) < 1e-5
        gx_bf, gk_bf = direct.causal_conv1d_bwd(g[b:b + 1], x[b:b + 1], k[b])
        assert rel_l2(gx_bf, xt.grad[b:b + 1]) < 1e-5
        assert rel_l2(gk_bf, kt.grad[b]) < 1e-5
