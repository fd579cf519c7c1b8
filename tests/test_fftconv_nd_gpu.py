"""GPU parity of the HIP 2D / 3D non-causal FFT conv against the CPU oracle.

Mirrors tests/ops/test_fftconv_custom.py (shared-kernel shapes, BLH, chunked
bitwise, FiLM per-sample kernels, bf16) and tests/ops/test_subq_ops_fft_conv2d.py
(3D vs 4D weight, non-square, batch one, odd channel counts), and
tests/ops/test_fftconv.py's 2D/3D backward checks; adds the BASELINE configs 4
and 5 on channel samples.  Tolerances: rel-L2 <= 1e-4 fp32, <= 2e-2 bf16 I/O.
"""

import os

import numpy as np
import pytest
import torch

from nvsubquadratic_amd import fftconv_hip as F
from oracle.fftconv_ref import fftconv_nd_np, fftconv_nd_torch, rel_l2


pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "nd.npz")

# The last two shapes leave less than half of an axis as padding (S > F/2: 60 -> F = 64, 50 -> 64), so the
# passes that fold a zero first-pass half run their unpruned variants too.
SHAPES_2D = [(2, 64, 32, 32, 7, 7), (4, 128, 14, 14, 7, 7), (2, 256, 28, 28, 13, 13), (1, 64, 64, 64, 15, 15),
             (1, 384, 14, 14, 14, 14), (2, 64, 14, 14, 28, 28), (2, 8, 32, 16, 7, 5), (1, 3, 5, 7, 10, 13),
             (2, 8, 60, 50, 3, 5), (1, 16, 20, 60, 9, 3)]


def _grad_check(xs, ks, fn, kb=1, dtype=torch.float32, tol=1e-4):
    torch.manual_seed(0)
    H = xs[1]
    x = torch.randn(*xs).to(dtype).requires_grad_(True)
    k = torch.randn(kb, H, *ks, requires_grad=True)
    s = torch.randn(H).to(dtype).requires_grad_(True)
    y_ref = fftconv_nd_torch(x, k, s)
    g = torch.randn_like(y_ref)
    y_ref.backward(g)
    xg = x.detach().cuda().requires_grad_(True)
    kg = k.detach().cuda().requires_grad_(True)
    sg = s.detach().cuda().requires_grad_(True)
    y = fn(xg, kg, sg)
    y.backward(g.cuda())
    assert y.dtype == dtype
    assert rel_l2(y_ref, y) < tol
    assert rel_l2(x.grad, xg.grad) < tol
    assert rel_l2(k.grad, kg.grad) < tol
    assert rel_l2(s.grad, sg.grad) < tol


@pytest.mark.parametrize("B,H,X,Y,Kx,Ky", SHAPES_2D)
def test_2d_shared_kernel_fwd_bwd(B, H, X, Y, Kx, Ky):
    _grad_check((B, H, X, Y), (Kx, Ky), F.fftconv2d_bhl)


@pytest.mark.parametrize("B,H,X,Y,Kx,Ky", [(2, 16, 32, 32, 7, 7), (3, 8, 14, 14, 14, 14)])
def test_2d_film_per_sample_kernel(B, H, X, Y, Kx, Ky):
    _grad_check((B, H, X, Y), (Kx, Ky), F.fftconv2d_bhl, kb=B)


def test_2d_film_per_sample_independence_bitwise():
    torch.manual_seed(1)
    x = torch.randn(3, 8, 16, 16, device="cuda")
    k = torch.randn(3, 8, 5, 5, device="cuda")
    y = F.fftconv2d_bhl(x, k)
    y1 = F.fftconv2d_bhl(x[1:2].contiguous(), k[1:2].contiguous())
    assert torch.equal(y[1:2], y1)


def test_2d_3d_and_4d_weight_equal_bitwise():
    torch.manual_seed(2)
    x = torch.randn(2, 8, 16, 16, device="cuda")
    k = torch.randn(8, 5, 5, device="cuda")
    assert torch.equal(F.fftconv2d_bhl(x, k), F.fftconv2d_bhl(x, k.unsqueeze(0)))


@pytest.mark.parametrize("chunk", [16, 32, 128])
def test_2d_chunked_bitwise(chunk):
    torch.manual_seed(3)
    x = torch.randn(2, 100, 14, 14, device="cuda")
    k = torch.randn(1, 100, 7, 7, device="cuda")
    s = torch.randn(100, device="cuda")
    assert torch.equal(F.fftconv2d_bhl(x, k, s), F.fftconv2d_bhl_chunked(x, k, s, chunk))


def test_2d_blh_matches():
    torch.manual_seed(4)
    x = torch.randn(2, 32, 32, 64)
    k = torch.randn(1, 7, 7, 64)
    y = F.fftconv2d_bhl_w_reshape(x.cuda(), k.cuda())
    y_ref = fftconv_nd_torch(x.permute(0, 3, 1, 2), k.permute(0, 3, 1, 2)).permute(0, 2, 3, 1)
    assert rel_l2(y_ref, y) < 1e-4
    assert torch.equal(y, F.fftconv2d_blh_chunked(x.cuda(), k.cuda(), chunk_size=16))


@pytest.mark.parametrize("H", [63, 65, 127, 255])
def test_2d_odd_channel_counts(H):
    torch.manual_seed(5)
    x = torch.randn(1, H, 16, 16)
    k = torch.randn(H, 5, 5)
    assert rel_l2(fftconv_nd_torch(x, k), F.fftconv2d_bhl(x.cuda(), k.cuda())) < 1e-4


def test_2d_bf16_io():
    _grad_check((2, 16, 32, 32), (9, 9), F.fftconv2d_bhl, dtype=torch.bfloat16, tol=2e-2)


@pytest.mark.parametrize("xs,ks", [((2, 4, 8, 8, 8), (3, 3, 3)), ((1, 3, 10, 9, 7), (5, 4, 3)),
                                   ((1, 2, 6, 6, 6), (12, 12, 12)), ((2, 2, 16, 8, 4), (7, 1, 3))])
def test_3d_fwd_bwd(xs, ks):
    _grad_check(xs, ks, F.fftconv3d_bhl)


# Shapes whose two inner axes fit one LDS plane (plane passes): F1 * F2/2 in
# {4096, 8192} with F1 >= 16, F2/2 >= 16; odd sizes, kernels longer than half the
# axis, and a kernel as long as twice the axis.
PLANE_3D = [((2, 3, 6, 100, 50), (5, 21, 27)), ((1, 2, 9, 64, 64), (4, 64, 64)), ((2, 2, 5, 33, 120), (3, 17, 9)),
            ((1, 2, 4, 20, 200), (3, 40, 5))]


@pytest.mark.parametrize("xs,ks", PLANE_3D)
def test_3d_plane_passes_fwd_bwd(xs, ks):
    _grad_check(xs, ks, F.fftconv3d_bhl)


def test_3d_plane_passes_film():
    _grad_check((2, 2, 6, 100, 50), (5, 21, 27), F.fftconv3d_bhl, kb=2)


# 128-point axis-0 columns take the wave-local adjoint (nd_col_bwd_w128_kernel): shared and per-sample filters,
# with (S0 <= 64) and without (S0 > 64) the zero-half fold, K0 > S0, and few channels (the batch loop split over
# workgroups, partial filter gradients summed afterwards).
W128_3D = [((3, 2, 100, 6, 8), (5, 3, 3), 1), ((2, 3, 64, 5, 9), (64, 3, 2), 1), ((2, 2, 100, 6, 8), (5, 3, 3), 2),
           ((1, 2, 40, 4, 4), (60, 2, 2), 1)]


@pytest.mark.parametrize("xs,ks,kb", W128_3D)
def test_3d_axis0_128_point_adjoint(xs, ks, kb):
    _grad_check(xs, ks, F.fftconv3d_bhl, kb=kb)


def test_3d_film_and_chunked():
    _grad_check((2, 3, 8, 8, 8), (5, 5, 5), F.fftconv3d_bhl, kb=2)
    torch.manual_seed(6)
    x = torch.randn(1, 40, 8, 8, 8, device="cuda")
    k = torch.randn(40, 3, 3, 3, device="cuda")
    assert torch.equal(F.fftconv3d_bhl(x, k), F.fftconv3d_bhl_chunked(x, k, chunk_size=16))


def test_golden_fixtures():
    d = np.load(GOLDEN)
    for i in range(int(d["n_nd"])):
        x = torch.tensor(d[f"n{i}_x"], dtype=torch.float32, device="cuda")
        k = torch.tensor(d[f"n{i}_k"], dtype=torch.float32, device="cuda")
        s = torch.tensor(d[f"n{i}_s"], dtype=torch.float32, device="cuda")
        fn = F.fftconv2d_bhl if x.ndim == 4 else F.fftconv3d_bhl
        assert rel_l2(d[f"n{i}_y"], fn(x, k, s)) < 1e-5, f"case {i}"


@pytest.mark.parametrize("xs,ks,kb", [((2, 3, 40, 24), (3, 17, 9), 1), ((2, 2, 12, 10, 14), (2, 5, 7, 6), 1),
                                       ((2, 2, 20, 16), (2 * 2, 9, 5), 2), ((2, 2, 6, 100, 50), (2, 5, 21, 27), 1)])
def test_backward_reusing_forward_state_is_bitwise_equal(xs, ks, kb):
    """A forward given a backward-sized workspace keeps x's transform and the filter
    spectrum; the backward reusing them equals the one that recomputes them, bitwise."""
    from nvsubquadratic_amd import _lib

    torch.manual_seed(21)
    nd = len(xs) - 2
    x = torch.randn(*xs, device="cuda")
    k = torch.randn(*ks, device="cuda")
    s = torch.randn(xs[1], device="cuda")
    g = torch.randn(*xs, device="cuda")
    lib = _lib.get_lib()
    S, K = _lib.i64_array(xs[2:]), _lib.i64_array(ks[1:])
    need = lib.nsq_fftconv_nd_workspace_bytes(nd, xs[0], xs[1], S, K, kb, _lib.NSQ_DIR_BWD)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    y = torch.empty_like(x)
    F.fftconv_nd_fwd_raw(x, k, s, y, kb, ws)
    outs = []
    for state, w in ((True, ws), (False, None)):
        gx, gk, gs = torch.empty_like(x), torch.empty_like(k), torch.empty(kb * xs[1], device="cuda")
        F.fftconv_nd_bwd_raw(g, x, k, s, gx, gk, gs, kb, w, fwd_state=state)
        outs.append((gx, gk, gs))
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    y2 = torch.empty_like(x)
    F.fftconv_nd_fwd_raw(x, k, s, y2, kb)  # minimum workspace: product in place
    assert torch.equal(y, y2)


def test_autograd_backward_receives_forward_state(monkeypatch):
    """Through autograd, the forward keeps its transforms and the backward reuses them
    (1D and ND): the backward launch is called with fwd_state=True."""
    seen = []
    real_1d, real_nd = F.causal_fftconv1d_bwd_raw, F.fftconv_nd_bwd_raw

    def spy_1d(*a, **kw):
        seen.append(("1d", kw.get("fwd_state")))
        return real_1d(*a, **kw)

    def spy_nd(*a, **kw):
        seen.append(("nd", kw.get("fwd_state")))
        return real_nd(*a, **kw)

    monkeypatch.setattr(F, "causal_fftconv1d_bwd_raw", spy_1d)
    monkeypatch.setattr(F, "fftconv_nd_bwd_raw", spy_nd)
    x1 = torch.randn(1, 2, 20000, device="cuda", requires_grad=True)
    k1 = torch.randn(1, 2, 20000, device="cuda", requires_grad=True)
    F.causal_fftconv1d_bhl(x1, k1).sum().backward()
    x2 = torch.randn(2, 3, 16, 12, device="cuda", requires_grad=True)
    k2 = torch.randn(3, 5, 7, device="cuda", requires_grad=True)
    F.fftconv2d_bhl(x2, k2).sum().backward()
    assert seen == [("1d", True), ("nd", True)]


def _radial_filter(C, size, sig_lo, sig_hi, nd, gen):
    sig = torch.empty(C).uniform_(sig_lo, sig_hi, generator=gen)
    ax = torch.arange(size).float() - size // 2
    grids = torch.meshgrid(*([ax] * nd), indexing="ij")
    r = torch.sqrt(sum(g ** 2 for g in grids))
    return torch.randn(C, *([size] * nd), generator=gen) * torch.exp(-r[None] / sig.view(-1, *([1] * nd)))


def test_config4_2d_channel_sample_bf16():
    """Config 4 (B=16, C=384, 128x128, bf16 I/O, radial filter) on 8 channels."""
    gen = torch.Generator().manual_seed(0)
    C = 8
    x = torch.randn(16, C, 128, 128, generator=gen).to(torch.bfloat16)
    k = _radial_filter(C, 128, 4.0, 64.0, 2, gen)
    s = torch.randn(C, generator=gen).to(torch.bfloat16)
    y = F.fftconv2d_bhl(x.cuda(), k.cuda(), s.cuda())
    assert y.dtype == torch.bfloat16
    assert rel_l2(fftconv_nd_torch(x, k, s), y) < 2e-2
    y64 = fftconv_nd_np(x.float().numpy(), k.numpy(), s.float().numpy())
    assert rel_l2(y64, y) < 5e-3


def test_config5_3d_channel_sample_bf16_fwd_bwd():
    """Config 5 (B=2, C=128, 64^3, bf16 I/O, radial filter) on 4 channels, forward and backward."""
    gen = torch.Generator().manual_seed(0)
    C = 4
    x = torch.randn(2, C, 64, 64, 64, generator=gen).to(torch.bfloat16).requires_grad_(True)
    k = _radial_filter(C, 64, 2.0, 32.0, 3, gen).requires_grad_(True)
    s = torch.randn(C, generator=gen).to(torch.bfloat16).requires_grad_(True)
    y_ref = fftconv_nd_torch(x, k, s)
    g = torch.randn(y_ref.shape, generator=gen).to(torch.bfloat16)
    y_ref.backward(g)
    xg, kg, sg = (t.detach().cuda().requires_grad_(True) for t in (x, k, s))
    y = F.fftconv3d_bhl(xg, kg, sg)
    y.backward(g.cuda())
    assert rel_l2(y_ref, y) < 2e-2
    assert rel_l2(x.grad, xg.grad) < 2e-2
    assert rel_l2(k.grad, kg.grad) < 2e-2
    assert rel_l2(s.grad, sg.grad) < 2e-2


def test_state_budget_zero_recomputes_bitwise(monkeypatch):
    """N-d: the backward without a kept forward state recomputes x's and the filter's spectra, bitwise equal."""
    torch.manual_seed(22)
    x = torch.randn(2, 4, 24, 20, device="cuda", requires_grad=True)
    k = torch.randn(1, 4, 7, 9, device="cuda", requires_grad=True)
    s = torch.randn(4, device="cuda", requires_grad=True)
    g = torch.randn(2, 4, 24, 20, device="cuda")
    grads = []
    for budget in (None, "0"):
        if budget is None:
            monkeypatch.delenv("NSQ_STATE_MAX_BYTES", raising=False)
        else:
            monkeypatch.setenv("NSQ_STATE_MAX_BYTES", budget)
        for t in (x, k, s):
            t.grad = None
        F.fftconv2d_bhl(x, k, s).backward(g)
        grads.append([t.grad.clone() for t in (x, k, s)])
    for a, b in zip(*grads):
        assert torch.equal(a, b)
