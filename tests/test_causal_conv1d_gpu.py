"""GPU parity of the HIP direct causal conv and B2B block against the CPU oracle.

Mirrors tests/ops/test_causal_conv1d_custom.py (forward :63-110 incl. bias and
silu; B2B shape/finite :112-133, here extended to values) and
tests/modules/test_subq_ops_causal_conv1d.py (module forward/backward and the
construction errors :74-148).  Tolerances: the reference's atol=1e-3/rtol=1e-4
elementwise for fp32 plus rel-L2 <= 1e-4 (fp32) / 2e-2 (bf16).
"""

import numpy as np
import os
import pytest
import torch

from nvsubquadratic_amd.causal_conv1d_hip import b2b_causal_conv1d, causal_conv1d
from nvsubquadratic_amd.modules import HipCausalConv1d
from oracle.direct_ref import b2b_causal_conv1d_torch, causal_conv1d_torch
from oracle.fftconv_ref import rel_l2


pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "direct1d.npz")


@pytest.mark.parametrize("C,L,K", [(16, 64, 3), (36, 256, 3), (64, 128, 7), (8, 5000, 128), (4, 3000, 256), (3, 7, 9)])
@pytest.mark.parametrize("with_bias", [False, True])
@pytest.mark.parametrize("act", ["identity", "silu"])
def test_forward_backward_vs_reference(C, L, K, with_bias, act):
    torch.manual_seed(42)
    x = torch.randn(2, C, L, requires_grad=True)
    w = torch.randn(C, K, requires_grad=True)
    b = torch.randn(C, requires_grad=True) if with_bias else None
    y_ref = causal_conv1d_torch(x, w, b, act)
    g = torch.randn_like(y_ref)
    y_ref.backward(g)
    xg = x.detach().cuda().requires_grad_(True)
    wg = w.detach().cuda().requires_grad_(True)
    bg = b.detach().cuda().requires_grad_(True) if with_bias else None
    y = causal_conv1d(xg, wg, bg, act)
    y.backward(g.cuda())
    torch.testing.assert_close(y.cpu(), y_ref, atol=1e-3, rtol=1e-4)
    assert rel_l2(y_ref, y) < 1e-4
    assert rel_l2(x.grad, xg.grad) < 1e-4
    assert rel_l2(w.grad, wg.grad) < 1e-4
    if with_bias:
        assert rel_l2(b.grad, bg.grad) < 1e-4


def test_golden_fixtures():
    d = np.load(GOLDEN)
    for i in range(int(d["n_direct"])):
        x, w, b = (torch.tensor(d[f"d{i}_{n}"], dtype=torch.float32, device="cuda") for n in ("x", "w", "b"))
        assert rel_l2(d[f"d{i}_y"], causal_conv1d(x, w, b)) < 1e-5
        assert rel_l2(d[f"d{i}_y_silu"], causal_conv1d(x, w, b, "silu")) < 1e-5
    for i in range(int(d["n_b2b"])):
        x, wp, wm, sk = (torch.tensor(d[f"b{i}_{n}"], dtype=torch.float32, device="cuda")
                         for n in ("x", "wp", "wm", "skip"))
        assert rel_l2(d[f"b{i}_y"], b2b_causal_conv1d(x, wp, wm, sk)) < 1e-5


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_low_precision_io(dtype):
    torch.manual_seed(1)
    x = torch.randn(2, 32, 700, dtype=dtype)
    w = torch.randn(32, 4)
    y = causal_conv1d(x.cuda(), w.cuda(), None, "silu")
    assert y.dtype == dtype
    assert rel_l2(causal_conv1d_torch(x.float(), w, None, "silu"), y) < 2e-2


def test_batch_and_tile_independence_bitwise():
    torch.manual_seed(2)
    x = torch.randn(3, 8, 5000, device="cuda")
    w = torch.randn(8, 31, device="cuda")
    y = causal_conv1d(x, w)
    y1 = causal_conv1d(x[1:2].contiguous(), w)
    assert torch.equal(y[1:2], y1)


@pytest.mark.parametrize("K", [2, 3, 4, 5, 8, 9, 17, 33, 128, 256])
def test_halo_before_row_start_reads_zero(K):
    """Outputs whose window reaches before position 0 see only the zero padding.

    Rows are staged through raw buffers; positions before the row start must read
    as zero however the compiler splits the element offset (a negative offset plus
    a folded immediate can wrap back into range).
    """
    torch.manual_seed(11)
    B, C, L = 3, 5, 300
    x = torch.randn(B, C, L, requires_grad=True)
    w = torch.randn(C, K, requires_grad=True)
    y_ref = causal_conv1d_torch(x, w, None)
    g = torch.randn_like(y_ref)
    y_ref.backward(g)
    xg, wg = x.detach().cuda().requires_grad_(True), w.detach().cuda().requires_grad_(True)
    y = causal_conv1d(xg, wg)
    y.backward(g.cuda())
    assert rel_l2(y_ref[..., :K], y[..., :K]) < 1e-5
    assert rel_l2(y_ref, y) < 1e-5
    assert rel_l2(x.grad, xg.grad) < 1e-5
    assert rel_l2(w.grad, wg.grad) < 1e-5


@pytest.mark.parametrize("K", [1, 2, 3, 4, 5, 6, 7, 8, 9, 12, 15, 16])
@pytest.mark.parametrize("L", [1, 13, 4103, 18432])
def test_short_taps_backward_across_tiles_and_batches(K, L):
    """Up to 16 taps the whole backward is one register-resident pass whose
    weight/bias partials cover runs of (batch, tile) pairs; with 3 batches and
    up to 9 tiles per row those runs cross row ends.  Ragged lengths take the
    element-load path, multiples of 8 the vector path."""
    torch.manual_seed(100 + K)
    B, C = 3, 6
    x = torch.randn(B, C, L, dtype=torch.float64, requires_grad=True)
    w = torch.randn(C, K, dtype=torch.float64, requires_grad=True)
    b = torch.randn(C, dtype=torch.float64, requires_grad=True)
    y_ref = causal_conv1d_torch(x, w, b, "silu")
    g = torch.randn_like(y_ref)
    y_ref.backward(g)
    xg = x.detach().float().cuda().requires_grad_(True)
    wg = w.detach().float().cuda().requires_grad_(True)
    bg = b.detach().float().cuda().requires_grad_(True)
    y = causal_conv1d(xg, wg, bg, "silu")
    y.backward(g.float().cuda())
    assert rel_l2(y_ref, y.double()) < 1e-5
    assert rel_l2(x.grad, xg.grad.double()) < 1e-5
    assert rel_l2(w.grad, wg.grad.double()) < 1e-5
    assert rel_l2(b.grad, bg.grad.double()) < 1e-5


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("K", [4, 7, 13])
def test_short_taps_backward_low_precision_io(dtype, K):
    torch.manual_seed(5)
    x = torch.randn(2, 16, 3000).to(dtype)
    w = torch.randn(16, K)
    b = torch.randn(16)
    xr = x.float().requires_grad_(True)
    wr, br = w.clone().requires_grad_(True), b.clone().requires_grad_(True)
    y_ref = causal_conv1d_torch(xr, wr, br, "silu")
    g = torch.randn_like(y_ref).to(dtype)
    y_ref.backward(g.float())
    xg = x.cuda().requires_grad_(True)
    wg, bg = w.cuda().requires_grad_(True), b.cuda().requires_grad_(True)
    y = causal_conv1d(xg, wg, bg, "silu")
    y.backward(g.cuda())
    assert xg.grad.dtype == dtype
    assert rel_l2(y_ref, y.float()) < 2e-2
    assert rel_l2(xr.grad, xg.grad.float()) < 2e-2
    assert rel_l2(wr.grad, wg.grad) < 2e-2
    assert rel_l2(br.grad, bg.grad) < 2e-2


@pytest.mark.parametrize("K", [15, 16, 17, 33, 34, 65, 66, 129, 130, 256])
@pytest.mark.parametrize("act", ["identity", "silu"])
def test_tap_counts_across_matrix_core_plans(K, act):
    """Direct conv above 16 taps runs as banded Toeplitz MFMA products (forward,
    the silu pre-activation gradient, the input-gradient correlation and the
    weight gradient, on bands of 12, 20, 36 or 68 steps); up to 16 taps the
    register-window kernels run.  Ragged length, bias, two batches; forward and
    gradients against a float64 reference."""
    torch.manual_seed(200 + K)
    B, C, L = 2, 3, 4700
    x = torch.randn(B, C, L, dtype=torch.float64, requires_grad=True)
    w = (torch.randn(C, K, dtype=torch.float64) / K ** 0.5).requires_grad_(True)
    b = torch.randn(C, dtype=torch.float64, requires_grad=True)
    y_ref = causal_conv1d_torch(x, w, b, act)
    g = torch.randn_like(y_ref)
    y_ref.backward(g)
    xg, wg, bg = (t.detach().float().cuda().requires_grad_(True) for t in (x, w, b))
    y = causal_conv1d(xg, wg, bg, act)
    y.backward(g.float().cuda())
    assert rel_l2(y_ref, y.detach().double()) < 1e-5
    assert rel_l2(y_ref[..., :K + 2], y.detach()[..., :K + 2].double()) < 1e-5
    for ref, got in ((x, xg), (w, wg), (b, bg)):
        assert rel_l2(ref.grad, got.grad.double()) < 1e-5
    assert rel_l2(x.grad[..., -K - 2:], xg.grad[..., -K - 2:].double()) < 1e-5


@pytest.mark.parametrize("Kp,Km", [(2, 3), (4, 4), (5, 7), (8, 1), (1, 9), (7, 33)])
def test_b2b_halo_before_row_start_reads_zero(Kp, Km):
    """B2B forward and backward near the row start for several halo widths."""
    torch.manual_seed(12)
    B, C, L = 2, 3, 200
    x = torch.randn(B, 3 * C, L, requires_grad=True)
    wp = torch.randn(3 * C, Kp, requires_grad=True)
    wm = torch.randn(C, Km, requires_grad=True)
    sk = torch.randn(C, requires_grad=True)
    y_ref = b2b_causal_conv1d_torch(x, wp, wm, sk)
    g = torch.randn_like(y_ref)
    y_ref.backward(g)
    args = [t.detach().cuda().requires_grad_(True) for t in (x, wp, wm, sk)]
    y = b2b_causal_conv1d(*args)
    y.backward(g.cuda())
    assert rel_l2(y_ref, y) < 1e-4
    assert rel_l2(x.grad[..., :Kp + Km], args[0].grad[..., :Kp + Km]) < 1e-4
    for ref, got in zip((x, wp, wm, sk), args):
        assert rel_l2(ref.grad, got.grad) < 1e-4


# --------------------------------------------------------------------------- B2B
@pytest.mark.parametrize("B,C,L,Kp,Km", [(2, 16, 64, 3, 3), (4, 32, 128, 4, 4), (2, 16, 128, 8, 8),
                                         (1, 8, 3000, 3, 128), (2, 4, 257, 5, 256)])
def test_b2b_forward_backward(B, C, L, Kp, Km):
    torch.manual_seed(42)
    x = torch.randn(B, 3 * C, L, requires_grad=True)
    wp = (torch.randn(3 * C, Kp) / Kp ** 0.5).requires_grad_(True)
    wm = (torch.randn(C, Km) / Km ** 0.5).requires_grad_(True)
    sk = torch.randn(C, requires_grad=True)
    y_ref = b2b_causal_conv1d_torch(x, wp, wm, sk)
    g = torch.randn_like(y_ref)
    y_ref.backward(g)
    args = [t.detach().cuda().requires_grad_(True) for t in (x, wp, wm, sk)]
    y = b2b_causal_conv1d(*args)
    assert y.shape == (B, C, L) and torch.isfinite(y).all()
    y.backward(g.cuda())
    assert rel_l2(y_ref, y) < 1e-4
    for ref, got in zip((x, wp, wm, sk), args):
        assert rel_l2(ref.grad, got.grad) < 1e-4


def test_b2b_backward_every_channel_many_workgroups():
    """The fused adjoint (projection taps <= 4, matrix-core mixer) with many workgroups per CU in
    flight, fp32, checked channel by channel: each thread's k / v windows read x words that
    other waves stage, so a missing barrier there corrupts runs of positions in a few
    channels only -- invisible in one rel-L2 over all channels, caught per row here."""
    torch.manual_seed(7)
    B, C, L, Kp, Km = 4, 512, 8192, 3, 128
    x = torch.randn(B, 3 * C, L, requires_grad=True)
    wp = (torch.randn(3 * C, Kp) / Kp ** 0.5).requires_grad_(True)
    wm = (torch.randn(C, Km) / Km ** 0.5).requires_grad_(True)
    sk = torch.randn(C, requires_grad=True)
    y_ref = b2b_causal_conv1d_torch(x, wp, wm, sk)
    g = torch.randn_like(y_ref)
    y_ref.backward(g)
    args = [t.detach().cuda().requires_grad_(True) for t in (x, wp, wm, sk)]
    b2b_causal_conv1d(*args).backward(g.cuda())
    gx = args[0].grad.cpu().double()
    rx = x.grad.double()
    err_x = ((gx - rx).norm(dim=2) / rx.norm(dim=2)).max().item()  # worst (batch, channel) row
    err_wp = ((args[1].grad.cpu().double() - wp.grad.double()).norm(dim=1) / wp.grad.double().norm(dim=1)).max().item()
    assert err_x < 1e-4, err_x
    assert err_wp < 1e-4, err_wp
    for ref, got in zip((wm, sk), args[2:]):
        assert rel_l2(ref.grad, got.grad) < 1e-4


@pytest.mark.parametrize("Km", [15, 16, 17, 33, 34, 65, 66, 128, 129, 130, 256])
def test_b2b_mixer_tap_counts_across_matrix_core_plans(Km):
    """Mixer tap counts on both sides of each matrix-core step-count boundary.

    From 16 taps the mixer conv (forward), its adjoint correlation and its
    weight gradient run as banded Toeplitz products on the matrix cores with
    12, 20, 36 or 68 steps (up to 33, 65, 129, 257 taps); 15 taps stay on the
    FMA loop.  Ragged length (not a multiple of the 2048-output tile), several
    batches, nonzero skip; forward and all four gradients against float64.
    """
    torch.manual_seed(100 + Km)
    B, C, L = 3, 5, 4500
    x = torch.randn(B, 3 * C, L, dtype=torch.float64, requires_grad=True)
    wp = (torch.randn(3 * C, 3, dtype=torch.float64) / 3 ** 0.5).requires_grad_(True)
    wm = (torch.randn(C, Km, dtype=torch.float64) / Km ** 0.5).requires_grad_(True)
    sk = torch.randn(C, dtype=torch.float64, requires_grad=True)
    # the B2B composition of the oracle's conv, in float64
    p = causal_conv1d_torch(x, wp)
    q, k, v = p[:, :C], p[:, C:2 * C], p[:, 2 * C:]
    z = k * v
    y_ref = q * (causal_conv1d_torch(z, wm) + sk.view(1, C, 1) * z)
    gy = torch.randn_like(y_ref)
    y_ref.backward(gy)
    args = [t.detach().float().cuda().requires_grad_(True) for t in (x, wp, wm, sk)]
    y = b2b_causal_conv1d(*args)
    y.backward(gy.float().cuda())
    y = y.detach().double().cpu()
    assert rel_l2(y_ref, y) < 1e-5
    # the first outputs of a row and of a tile see the causal zero padding / the tile halo
    assert rel_l2(y_ref[..., :Km + 3], y[..., :Km + 3]) < 1e-5
    assert rel_l2(y_ref[..., 2048:2048 + Km], y[..., 2048:2048 + Km]) < 1e-5
    for ref, got in zip((x, wp, wm, sk), args):
        assert rel_l2(ref.grad, got.grad.double()) < 1e-5
    # gradients near the row end and across a tile boundary
    assert rel_l2(x.grad[..., -Km - 3:], args[0].grad[..., -Km - 3:].double()) < 1e-5
    assert rel_l2(x.grad[..., 2040:2060], args[0].grad[..., 2040:2060].double()) < 1e-5


def test_b2b_config2_shape_bf16_sample():
    """Config 2 (B=4, L=8192, 3*4096 channels, k=3 then k=128) on a channel sample, bf16 I/O."""
    torch.manual_seed(3)
    B, C, L = 4, 64, 8192
    x = torch.randn(B, 3 * C, L).to(torch.bfloat16)
    wp = torch.randn(3 * C, 3)
    wm = torch.randn(C, 128) / 128 ** 0.5
    sk = torch.zeros(C)
    y = b2b_causal_conv1d(x.cuda(), wp.cuda(), wm.cuda(), sk.cuda())
    assert y.dtype == torch.bfloat16
    assert rel_l2(b2b_causal_conv1d_torch(x.float(), wp, wm, sk), y) < 2e-2


# --------------------------------------------------------------------------- module
@pytest.mark.parametrize("C,L,K", [(36, 256, 3), (64, 512, 7), (16, 128, 4)])
def test_module_matches_reference_conv(C, L, K):
    torch.manual_seed(42)
    ref = torch.nn.Conv1d(C, C, K, groups=C, bias=True)
    fast = HipCausalConv1d(C, C, K, groups=C, bias=True).cuda()
    fast.load_state_dict(ref.state_dict())
    x = torch.randn(2, C, L, requires_grad=True)
    y_ref = causal_conv1d_torch(x, ref.weight.squeeze(1), ref.bias)
    y_ref.sum().backward()
    xg = x.detach().cuda().requires_grad_(True)
    y = fast(xg)
    y.sum().backward()
    torch.testing.assert_close(y.cpu(), y_ref, atol=1e-3, rtol=1e-4)
    torch.testing.assert_close(xg.grad.cpu(), x.grad, atol=1e-2, rtol=1e-3)
    torch.testing.assert_close(fast.weight.grad.cpu(), ref.weight.grad, atol=1e-2, rtol=1e-3)
    torch.testing.assert_close(fast.bias.grad.cpu(), ref.bias.grad, atol=1e-2, rtol=1e-3)


@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, 4e-3), (torch.float16, 5e-4)])
@pytest.mark.parametrize("Km", [16, 33, 34, 65, 66, 128, 129, 256])
def test_b2b_16bit_io_mixer_as_bf16_products(dtype, tol, Km):
    """16-bit I/O runs the B2B mixer on v_mfma_f32_16x16x32_bf16 with z and the taps split into bf16
    halves (three products per step, ~2^-17 relative per product).  Against float64 of the same
    16-bit inputs the error is the output rounding: ~1e-3 (bf16) and ~1.5e-4 (fp16) rel-L2; a band
    or split mistake (a lost lo term alone is ~2^-9) fails the fp16 bound.  Tap counts on both sides
    of every band step boundary, ragged length, nonzero skip, the row start and a tile halo."""
    torch.manual_seed(200 + Km)
    B, C, L = 3, 5, 4500
    x = torch.randn(B, 3 * C, L).to(dtype)
    wp = torch.randn(3 * C, 3) / 3 ** 0.5
    wm = torch.randn(C, Km) / Km ** 0.5
    sk = torch.randn(C)
    p = causal_conv1d_torch(x.double(), wp.double())
    q, k, v = p[:, :C], p[:, C:2 * C], p[:, 2 * C:]
    z = k * v
    y64 = q * (causal_conv1d_torch(z, wm.double()) + sk.double().view(1, C, 1) * z)
    y = b2b_causal_conv1d(x.cuda(), wp.cuda(), wm.cuda(), sk.cuda())
    assert y.dtype == dtype
    y = y.double().cpu()
    assert rel_l2(y64, y) < tol
    assert rel_l2(y64[..., :Km + 3], y[..., :Km + 3]) < tol
    assert rel_l2(y64[..., 2048:2048 + Km], y[..., 2048:2048 + Km]) < tol
