"""GPU parity of the HIP circular and mixed-boundary FFT conv against the CPU oracle.

Mirrors tests/ops/test_circular_fftconv.py (1D/2D/3D vs the spatial reference,
shortcut, dtype preservation, BLH layout, batched kernel, backward) and
tests/ops/test_mixed_fftconv.py (every per-axis combination, uniform cases
routed to the zero-padded / circular ops, chunked, impulse and DC responses,
backward).  Periodic lengths are powers of two (the HIP kernels' range; below
16 points on the periodic extension at FFT length 16, covered by the reference's
own 8-point shapes and 1/2/4-point ones): the reference's 12- and 48-point
periodic cases are replaced by 16- and 64-point ones, and non-power-of-two
sizes are checked to raise.
Tolerances: rel-L2 <= 1e-4 fp32, <= 2e-2 bf16 / fp16 I/O.
"""

import itertools

import numpy as np
import pytest
import torch

from nvsubquadratic_amd import circular_fftconv_hip as C
from nvsubquadratic_amd import fftconv_hip as Z
from nvsubquadratic_amd import mixed_fftconv_hip as M
from oracle.circular_ref import (circular_conv_direct_np, circular_fftconv_torch, mixed_conv_direct_np,
                                 mixed_fftconv_torch)
from oracle.fftconv_ref import rel_l2


pytestmark = pytest.mark.gpu

CIRC_FNS = {1: C.circular_fftconv1d_fp32_bhl, 2: C.circular_fftconv2d_fp32_bhl, 3: C.circular_fftconv3d_fp32_bhl}
MIXED_FNS = {1: M.mixed_fftconv1d_fp32_bhl, 2: M.mixed_fftconv2d_fp32_bhl, 3: M.mixed_fftconv3d_fp32_bhl}


def _fwd_bwd_check(xs, ks, fn, ref_fn, kb=1, dtype=torch.float32, tol=1e-4, shortcut=True):
    """Forward and x / kernel / shortcut gradients of `fn` (GPU) against `ref_fn` (CPU autograd; the
    references below compute in float64, the exact-math side of the tolerance)."""
    torch.manual_seed(0)
    H = xs[1]
    x = torch.randn(*xs).to(dtype).requires_grad_(True)
    k = torch.randn(kb, H, *ks, requires_grad=True)
    s = torch.randn(H).to(dtype).requires_grad_(True) if shortcut else None
    y_ref = ref_fn(x, k, s)
    g = torch.randn_like(y_ref)
    y_ref.backward(g)
    xg = x.detach().cuda().requires_grad_(True)
    kg = k.detach().cuda().requires_grad_(True)
    sg = s.detach().cuda().requires_grad_(True) if shortcut else None
    y = fn(xg, kg, sg)
    y.backward(g.cuda())
    assert y.dtype == dtype and y.shape == x.shape
    assert rel_l2(y_ref, y) < tol
    assert rel_l2(x.grad, xg.grad) < tol
    assert rel_l2(k.grad, kg.grad) < tol
    if shortcut:
        assert rel_l2(s.grad, sg.grad) < tol


def _circ64(x, k, s=None):
    return circular_fftconv_torch(x, k, s, compute_dtype=torch.float64)


# --- circular: forward vs the float64 brute force ---------------------------
CIRC_1D = [(2, 16, 64, 7), (2, 32, 128, 32), (1, 8, 256, 256), (4, 16, 64, 15), (2, 8, 16, 1), (1, 4, 16384, 100),
           (3, 5, 1024, 4), (2, 3, 8, 8), (2, 3, 8, 3), (1, 2, 4, 4), (1, 2, 2, 2), (2, 2, 1, 1)]
CIRC_2D = [(2, 8, 32, 32, 7, 7), (2, 16, 64, 64, 15, 15), (1, 8, 32, 32, 32, 32), (4, 8, 16, 16, 5, 5),
           (1, 4, 16, 128, 4, 9), (2, 3, 256, 32, 1, 32), (4, 6, 8, 8, 5, 5), (2, 3, 8, 8, 8, 8), (1, 2, 2, 64, 2, 7),
           (2, 2, 16, 4, 6, 3), (1, 2, 1, 16, 1, 5)]
CIRC_3D = [(2, 4, 16, 16, 16, 5, 5, 5), (1, 8, 16, 16, 16, 3, 3, 3), (2, 4, 16, 16, 16, 16, 16, 16),
           (1, 2, 32, 16, 64, 4, 7, 2), (1, 4, 8, 8, 8, 3, 3, 3), (2, 3, 8, 8, 8, 8, 8, 8), (1, 2, 4, 16, 2, 3, 5, 2)]


@pytest.mark.parametrize("B,H,L,K", CIRC_1D)
def test_circular_1d_vs_brute_force(B, H, L, K):
    rng = np.random.default_rng(B * 100 + K)
    x = rng.standard_normal((B, H, L)).astype(np.float32)
    k = rng.standard_normal((1, H, K)).astype(np.float32)
    y = C.circular_fftconv1d_fp32_bhl(torch.tensor(x).cuda(), torch.tensor(k).cuda())
    assert rel_l2(circular_conv_direct_np(x, k), y) < 1e-4


@pytest.mark.parametrize("B,H,X,Y,Kx,Ky", CIRC_2D)
def test_circular_2d_vs_brute_force(B, H, X, Y, Kx, Ky):
    rng = np.random.default_rng(X + Kx)
    x = rng.standard_normal((B, H, X, Y)).astype(np.float32)
    k = rng.standard_normal((1, H, Kx, Ky)).astype(np.float32)
    y = C.circular_fftconv2d_fp32_bhl(torch.tensor(x).cuda(), torch.tensor(k).cuda())
    ref = circular_conv_direct_np(x, k) if Kx * Ky <= 256 else _circ64(torch.tensor(x), torch.tensor(k))
    assert rel_l2(ref, y) < 1e-4


@pytest.mark.parametrize("B,H,X,Y,Z,Kx,Ky,Kz", CIRC_3D)
def test_circular_3d_vs_brute_force(B, H, X, Y, Z, Kx, Ky, Kz):
    rng = np.random.default_rng(X + Kx + Kz)
    x = rng.standard_normal((B, H, X, Y, Z)).astype(np.float32)
    k = rng.standard_normal((1, H, Kx, Ky, Kz)).astype(np.float32)
    y = C.circular_fftconv3d_fp32_bhl(torch.tensor(x).cuda(), torch.tensor(k).cuda())
    big = Kx * Ky * Kz > 256
    ref = _circ64(torch.tensor(x), torch.tensor(k)) if big else circular_conv_direct_np(x, k)
    assert rel_l2(ref, y) < 1e-4


# --- circular: backward, shortcut, FiLM, dtypes -----------------------------
@pytest.mark.parametrize("xs,ks", [((2, 8, 64), (15,)), ((1, 16, 128), (7,)), ((2, 4, 4096), (4096,)),
                                   ((2, 4, 16, 16), (5, 5)), ((1, 8, 32, 32), (7, 7)), ((2, 3, 64, 16), (6, 16)),
                                   ((2, 4, 16, 16, 16), (5, 5, 5)), ((1, 2, 16, 32, 16), (4, 1, 16)),
                                   ((2, 3, 8), (5,)), ((2, 4, 8, 8), (5, 4)), ((2, 3, 8, 8, 8), (3, 3, 3)),
                                   ((1, 4, 8, 8, 8), (3, 3, 3)), ((2, 2, 4, 32), (3, 9))])
def test_circular_fwd_bwd_vs_oracle(xs, ks):
    _fwd_bwd_check(xs, ks, CIRC_FNS[len(xs) - 2], _circ64)


@pytest.mark.parametrize("xs,ks", [((3, 8, 256), (9,)), ((2, 4, 32, 32), (5, 6)), ((2, 2, 16, 16, 32), (3, 4, 5)),
                                   ((3, 2, 8), (4,)), ((2, 3, 8, 8, 8), (5, 4, 3))])
def test_circular_film_per_sample_kernel(xs, ks):
    _fwd_bwd_check(xs, ks, CIRC_FNS[len(xs) - 2], _circ64, kb=xs[0])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("xs,ks", [((2, 8, 512), (31,)), ((2, 4, 32, 64), (7, 5)), ((1, 4, 16, 16, 16), (3, 3, 3))])
def test_circular_low_precision_io(dtype, xs, ks):
    _fwd_bwd_check(xs, ks, CIRC_FNS[len(xs) - 2], _circ64, dtype=dtype, tol=2e-2)


@pytest.mark.parametrize("nd", [1, 2, 3])
def test_circular_no_shortcut_and_w_reshape(nd):
    torch.manual_seed(4)
    S = {1: (256,), 2: (32, 16), 3: (16, 16, 16)}[nd]
    K = {1: (10,), 2: (5, 4), 3: (3, 4, 5)}[nd]
    x = torch.randn(2, 6, *S, device="cuda")
    k = torch.randn(1, 6, *K, device="cuda")
    y = CIRC_FNS[nd](x, k)
    assert rel_l2(_circ64(x.cpu(), k.cpu()), y) < 1e-4
    wr = {1: C.circular_fftconv1d_fp32_bhl_w_reshape, 2: C.circular_fftconv2d_fp32_bhl_w_reshape,
          3: C.circular_fftconv3d_fp32_bhl_w_reshape}[nd]
    perm = (0,) + tuple(range(2, 2 + nd)) + (1,)
    y_blh = wr(x.permute(perm).contiguous(), k.permute(perm).contiguous())
    assert torch.equal(y_blh, y.permute(perm))
    # use_phase_shift=False selects the reference's spatial roll; the result is the same
    assert torch.equal(CIRC_FNS[nd](x, k, use_phase_shift=False), y)


def test_circular_dc_and_impulse_response():
    torch.manual_seed(5)
    k = torch.randn(1, 4, 5, 5, device="cuda")
    y = C.circular_fftconv2d_fp32_bhl(torch.ones(2, 4, 16, 16, device="cuda"), k)
    torch.testing.assert_close(y, k.sum(dim=(-1, -2)).view(1, 4, 1, 1).expand_as(y), rtol=1e-5, atol=1e-5)
    x = torch.zeros(1, 4, 16, 16, device="cuda")
    x[..., 0, 0] = 1.0
    y = C.circular_fftconv2d_fp32_bhl(x, k)
    torch.testing.assert_close(y.cpu(), torch.tensor(circular_conv_direct_np(x.cpu(), k.cpu()), dtype=torch.float32),
                               rtol=1e-6, atol=1e-6)


def test_circular_rejects_mismatched_shortcut_dtype():
    x = torch.randn(1, 4, 64, device="cuda")
    k = torch.randn(1, 4, 5, device="cuda")
    with pytest.raises(AssertionError):
        C.circular_fftconv1d_fp32_bhl(x, k, torch.randn(4, device="cuda", dtype=torch.bfloat16))


@pytest.mark.parametrize("xs,ks", [((1, 2, 2**25), (5,)), ((1, 2, 2048, 16), (3, 3)), ((1, 2, 1000, 12), (101, 3))])
def test_circular_unsupported_lengths_raise(xs, ks):
    """Out-of-range periodic lengths are refused, not approximated (1D: beyond the 4-step plan's 2^24; 1000 with
    101 taps: its periodic extension needs FFT length 2048 on that axis)."""
    x = torch.randn(*xs, device="cuda")
    k = torch.randn(1, xs[1], *ks, device="cuda")
    with pytest.raises(NotImplementedError):
        CIRC_FNS[len(xs) - 2](x, k)


# --- mixed boundary conditions -----------------------------------------------
COMBOS_2D = [p for p in itertools.product((False, True), repeat=2)]
COMBOS_3D = [p for p in itertools.product((False, True), repeat=3)]


@pytest.mark.parametrize("periodic", COMBOS_2D)
@pytest.mark.parametrize("B,H,X,Y,Kx,Ky", [(2, 8, 32, 32, 5, 5), (1, 16, 64, 64, 7, 9), (2, 8, 32, 32, 32, 32)])
def test_mixed_2d_vs_brute_force(periodic, B, H, X, Y, Kx, Ky):
    rng = np.random.default_rng(X + Kx)
    x = rng.standard_normal((B, H, X, Y)).astype(np.float32)
    k = rng.standard_normal((1, H, Kx, Ky)).astype(np.float32)
    y = M.mixed_fftconv2d_fp32_bhl(torch.tensor(x).cuda(), torch.tensor(k).cuda(), periodic)
    big = Kx * Ky > 256
    ref = (mixed_fftconv_torch(torch.tensor(x), torch.tensor(k), periodic, compute_dtype=torch.float64) if big
           else mixed_conv_direct_np(x, k, periodic))
    assert rel_l2(ref, y) < 1e-4


@pytest.mark.parametrize("periodic", COMBOS_3D)
@pytest.mark.parametrize("B,H,X,Y,Z,Kx,Ky,Kz", [(2, 4, 16, 16, 16, 5, 5, 5), (1, 8, 16, 16, 32, 7, 7, 5),
                                                (1, 4, 8, 8, 8, 5, 5, 5)])
def test_mixed_3d_vs_brute_force(periodic, B, H, X, Y, Z, Kx, Ky, Kz):
    rng = np.random.default_rng(X + Kx + Z)
    x = rng.standard_normal((B, H, X, Y, Z)).astype(np.float32)
    k = rng.standard_normal((1, H, Kx, Ky, Kz)).astype(np.float32)
    y = M.mixed_fftconv3d_fp32_bhl(torch.tensor(x).cuda(), torch.tensor(k).cuda(), periodic)
    assert rel_l2(mixed_fftconv_torch(torch.tensor(x), torch.tensor(k), periodic, compute_dtype=torch.float64), y) < 1e-4


@pytest.mark.parametrize("periodic", [(True, False), (False, True), (True, True)])
@pytest.mark.parametrize("xs,ks", [((2, 4, 16, 32), (5, 40)), ((1, 8, 64, 16), (7, 7))])
def test_mixed_2d_fwd_bwd(periodic, xs, ks):
    ks = tuple(min(kd, sd) if p else kd for kd, sd, p in zip(ks, xs[2:], periodic))
    _fwd_bwd_check(xs, ks, lambda x, k, s: M.mixed_fftconv2d_fp32_bhl(x, k, periodic, s),
                   lambda x, k, s: mixed_fftconv_torch(x, k, periodic, s, compute_dtype=torch.float64))


@pytest.mark.parametrize("periodic", [(True, False, True), (False, True, False)])
def test_mixed_3d_fwd_bwd_film(periodic):
    _fwd_bwd_check((2, 3, 16, 32, 16), (3, 6, 4), lambda x, k, s: M.mixed_fftconv3d_fp32_bhl(x, k, periodic, s),
                   lambda x, k, s: mixed_fftconv_torch(x, k, periodic, s, compute_dtype=torch.float64), kb=2)


def test_mixed_uniform_cases_route_to_zero_and_circular_ops():
    torch.manual_seed(6)
    x = torch.randn(2, 8, 32, 32, device="cuda")
    k = torch.randn(1, 8, 5, 7, device="cuda")
    assert torch.equal(M.mixed_fftconv2d_fp32_bhl(x, k, (False, False)), Z.fftconv2d_bhl(x, k))
    assert torch.equal(M.mixed_fftconv2d_fp32_bhl(x, k, (True, True)), C.circular_fftconv2d_fp32_bhl(x, k))
    x1 = torch.randn(2, 8, 128, device="cuda")
    k1 = torch.randn(1, 8, 9, device="cuda")
    assert torch.equal(M.mixed_fftconv1d_fp32_bhl(x1, k1, (True,)), C.circular_fftconv1d_fp32_bhl(x1, k1))
    assert torch.equal(M.mixed_fftconv1d_fp32_bhl(x1, k1, (False,)), Z.fftconv1d_bhl(x1, k1))


@pytest.mark.parametrize("periodic", COMBOS_2D)
def test_mixed_chunked_and_w_reshape_bitwise(periodic):
    torch.manual_seed(7)
    x = torch.randn(2, 40, 16, 32, device="cuda")
    k = torch.randn(1, 40, 5, 4, device="cuda")
    s = torch.randn(40, device="cuda")
    y = M.mixed_fftconv2d_fp32_bhl(x, k, periodic, s)
    assert torch.equal(M.mixed_fftconv2d_fp32_bhl_chunked(x, k, periodic, s, chunk_size=16), y)
    y_blh = M.mixed_fftconv2d_fp32_bhl_w_reshape(x.permute(0, 2, 3, 1).contiguous(), k.permute(0, 2, 3, 1).contiguous(),
                                                 periodic, s)
    assert torch.equal(y_blh, y.permute(0, 2, 3, 1))
    y_blh_c = M.mixed_fftconv2d_fp32_bhl_w_reshape_chunked(x.permute(0, 2, 3, 1).contiguous(),
                                                           k.permute(0, 2, 3, 1).contiguous(), periodic, s,
                                                           chunk_size=16)
    assert torch.equal(y_blh_c, y.permute(0, 2, 3, 1))


@pytest.mark.parametrize("periodic", COMBOS_3D)
def test_mixed_impulse_response_3d(periodic):
    """tests/ops/test_mixed_fftconv.py:666-676 (8^3, K = 3 x 5 x 4)."""
    torch.manual_seed(0)
    x = torch.zeros(1, 2, 8, 8, 8, device="cuda")
    x[..., 0, 0, 0] = 1.0
    k = torch.randn(1, 2, 3, 5, 4, device="cuda")
    y = M.mixed_fftconv3d_fp32_bhl(x, k, periodic)
    ref = torch.tensor(mixed_conv_direct_np(x.cpu(), k.cpu(), periodic), dtype=torch.float32)
    torch.testing.assert_close(y.cpu(), ref, rtol=1e-6, atol=1e-6)


def test_mixed_periodic_kernel_larger_than_axis_rejected():
    x = torch.randn(1, 2, 16, 16, device="cuda")
    with pytest.raises(AssertionError):
        M.mixed_fftconv2d_fp32_bhl(x, torch.randn(1, 2, 17, 3, device="cuda"), (True, False))


@pytest.mark.parametrize("periodic", [(True, False), (False, True)])
def test_mixed_2d_short_periodic_fwd_bwd(periodic):
    """gray_scott / MHD-like token grids: an 8-point periodic axis beside a zero-padded one."""
    xs = (2, 4, 8, 16) if periodic[0] else (2, 4, 16, 8)
    ks = (5, 31) if periodic[0] else (31, 8)
    _fwd_bwd_check(xs, ks, lambda x, k, s: M.mixed_fftconv2d_fp32_bhl(x, k, periodic, s),
                   lambda x, k, s: mixed_fftconv_torch(x, k, periodic, s, compute_dtype=torch.float64))


def test_dc_response_all_periodic_3d_short():
    """tests/ops/test_mixed_fftconv.py:697: constant input -> sum(kernel) everywhere (8^3)."""
    torch.manual_seed(0)
    k = torch.randn(1, 2, 5, 5, 5, device="cuda")
    y = M.mixed_fftconv3d_fp32_bhl(torch.ones(1, 2, 8, 8, 8, device="cuda"), k, (True, True, True))
    torch.testing.assert_close(y, k.sum(dim=(-1, -2, -3)).view(1, 2, 1, 1, 1).expand_as(y), rtol=1e-5, atol=1e-5)


# --- periodic axes whose length is not a power of two ------------------------
# Run as zero-padded axes on the periodic extension of x; the oracle (float64 and the reference's
# float32 arithmetic) takes any length through torch.fft, and is pinned to the brute force on
# non-power-of-two lengths by the CPU tests.
NPOW2 = [((2, 3, 48), (1, 3, 5), (True,)), ((1, 2, 1000), (1, 2, 30), (True,)), ((2, 2, 12), (2, 2, 12), (True,)),
         ((2, 3, 24, 20), (1, 3, 5, 6), (True, True)), ((1, 2, 48, 16), (1, 2, 7, 4), (True, True)),
         ((2, 2, 12, 10, 8), (1, 2, 3, 4, 5), (True, True, True)),
         ((2, 2, 24, 20), (1, 2, 5, 7), (True, False)), ((1, 3, 16, 12), (1, 3, 20, 5), (False, True)),
         ((1, 2, 6, 16, 10), (1, 2, 3, 8, 4), (True, True, False)), ((1, 2, 224, 9), (1, 2, 31, 3), (True, False))]


@pytest.mark.parametrize("xs,ks,per", NPOW2)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_periodic_non_power_of_two_fwd_bwd(xs, ks, per, dtype):
    torch.manual_seed(sum(xs) + sum(ks))
    x = torch.randn(*xs).to(dtype).requires_grad_(True)
    k = torch.randn(*ks).requires_grad_(True)
    s = torch.randn(xs[1]).to(dtype).requires_grad_(True)
    y_ref = mixed_fftconv_torch(x, k, per, s)
    g = torch.randn_like(y_ref)
    y_ref.backward(g)
    xg, kg, sg = (t.detach().cuda().requires_grad_(True) for t in (x, k, s))
    nd = len(xs) - 2
    fn = CIRC_FNS[nd] if all(per) else None
    y = fn(xg, kg, sg) if fn else (M.mixed_fftconv1d_fp32_bhl, M.mixed_fftconv2d_fp32_bhl,
                                   M.mixed_fftconv3d_fp32_bhl)[nd - 1](xg, kg, per, sg)
    y.backward(g.cuda())
    assert y.dtype == dtype and y.shape == y_ref.shape
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    assert rel_l2(y_ref, y) < tol
    for a, b in ((x, xg), (k, kg), (s, sg)):
        assert rel_l2(a.grad, b.grad) < tol
    if dtype == torch.float32:
        y64 = mixed_fftconv_torch(x.detach().double(), k.detach().double(), per, s.detach().double(),
                                  compute_dtype=torch.float64)
        assert rel_l2(y64, y) < 1e-5
