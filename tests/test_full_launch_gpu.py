"""GPU parity of the benchmarked launches themselves, at their full sizes.

The benchmark times configs 2-5 at full size, and several kernels choose their
work split from the launch size: the axis-0 product pass of the 2D/3D engine
gives one workgroup a run of ceil(B / bsplit) images (prefetching the next
image's columns while the current one transforms) and the adjoint pass loops
over its images in the same way.  Channel samples of a config run a different
split than the full config, so here the op runs on the full tensors and a few
channels (first, last and two inner ones, all images) are compared with the
oracle on those channels only.  Each op is depthwise, so a channel's outputs
and gradients depend on that channel's inputs alone.

Which split each test reaches (axis0_batch_split in csrc/fftconv_nd.hip,
mirrored by :func:`_images_per_workgroup` and asserted below so a change of
the heuristic cannot silently move a test off the path it is meant for):

* config 4 (B=16, C=384, 128^2, filter 128^2, F = 256^2): product pass 8
  images per workgroup, adjoint 16;
* config 5 (B=2, C=128, 64^3, F = 128^3): 2 images per workgroup both ways;
* 2D B=2, H=2048, 32^2, filter 32^2 (F = 64^2): bsplit = 1, 2 images per
  workgroup both ways;
* 2D B=8, H=512, 64^2, filter 64^2 (F = 128^2): product bsplit = 3, runs of
  3, 3 and 2 images; adjoint 8 images.

Tolerances: rel-L2 <= 1e-4 fp32, <= 2e-2 bf16 I/O against the float32 oracle,
plus a 5e-3 check of bf16 outputs against the float64 restatement.
"""

import math

import pytest
import torch

from nvsubquadratic_amd import fftconv_hip as F
from nvsubquadratic_amd.causal_conv1d_hip import b2b_causal_conv1d
from nvsubquadratic_amd.workloads import causal1d_case_fast, radial_filter
from oracle.direct_ref import b2b_causal_conv1d_torch
from oracle.fftconv_ref import causal_fftconv1d_np, causal_fftconv1d_torch, fftconv_nd_np, fftconv_nd_torch, rel_l2


pytestmark = pytest.mark.gpu


def _images_per_workgroup(B, H, S, K, adjoint):
    """Images one axis-0 workgroup runs for a shared filter on zero-padded axes."""
    nd = len(S)
    Fs = [max(16, 1 << math.ceil(math.log2(s + (k + 1) // 2))) for s, k in zip(S, K)]
    inner = Fs[-1] // 2 if nd == 2 else Fs[1] * (Fs[2] // 2 + 1)
    target, lo, want_total = (4096, 1024, 3072) if adjoint else (8192, 4096, 6144)
    m = min(16, max(4, target >> int(math.log2(Fs[0]))))
    blocks = inner // m + ((inner - inner // m * m) + 3) // 4
    wgs = H * blocks
    bsplit = 1 if wgs >= lo else min(-(-want_total // wgs), B)
    return -(-B // bsplit)


def _sampled(H):
    return sorted({0, 1, H // 2 + 1, H - 1})


def _nd_full_case(B, H, S, K, dtype, gen, sig=(4.0, 64.0)):
    x = torch.randn(B, H, *S, generator=gen).to(dtype)
    k = radial_filter(H, K[0], sig[0], sig[1], len(S), gen) if len(set(K)) == 1 else torch.randn(H, *K, generator=gen)
    s = torch.randn(H, generator=gen).to(dtype)
    g = torch.randn(B, H, *S, generator=gen).to(dtype)
    return x, k, s, g


def _check_nd_full(x, k, s, g, fn, tol, tol64=None):
    """Full-size HIP fwd+bwd; sampled channels against the oracle."""
    xg, kg, sg = (t.cuda().requires_grad_(True) for t in (x, k, s))
    y = fn(xg, kg, sg)
    y.backward(g.cuda())
    torch.cuda.synchronize()
    ch = _sampled(x.shape[1])
    xs = x[:, ch].clone().requires_grad_(True)
    ks = k[ch].clone().requires_grad_(True)
    ss = s[ch].clone().requires_grad_(True)
    y_ref = fftconv_nd_torch(xs, ks, ss)
    y_ref.backward(g[:, ch])
    assert y.dtype == x.dtype
    assert rel_l2(y_ref, y[:, ch]) < tol
    assert rel_l2(xs.grad, xg.grad[:, ch]) < tol
    assert rel_l2(ks.grad, kg.grad[ch]) < tol
    assert rel_l2(ss.grad, sg.grad[ch]) < tol
    if tol64 is not None:
        y64 = fftconv_nd_np(x[:, ch].float().numpy(), k[ch].numpy(), s[ch].float().numpy())
        assert rel_l2(y64, y[:, ch]) < tol64


@pytest.mark.parametrize("B,H,S,K,fwd_imgs,bwd_imgs", [
    (2, 2048, (32, 32), (32, 32), 2, 2),  # bsplit = 1 both ways
    (8, 512, (64, 64), (64, 64), 3, 8),   # product pass runs of 3, 3, 2 images
])
def test_2d_multi_image_axis0_workgroups_fp32(B, H, S, K, fwd_imgs, bwd_imgs):
    assert _images_per_workgroup(B, H, S, K, adjoint=False) == fwd_imgs
    assert _images_per_workgroup(B, H, S, K, adjoint=True) == bwd_imgs
    gen = torch.Generator().manual_seed(31)
    x, k, s, g = _nd_full_case(B, H, S, K, torch.float32, gen)
    _check_nd_full(x, k, s, g, F.fftconv2d_bhl, 1e-4)


def test_config4_full_launch_bf16():
    """Config 4 at full size: B=16, C=384, 128^2 bf16, radial filter sigma ~ U(4, 64)."""
    B, C, S = 16, 384, (128, 128)
    assert _images_per_workgroup(B, C, S, S, adjoint=False) == 8
    assert _images_per_workgroup(B, C, S, S, adjoint=True) == 16
    gen = torch.Generator().manual_seed(0)
    x, k, s, g = _nd_full_case(B, C, S, S, torch.bfloat16, gen, sig=(4.0, 64.0))
    _check_nd_full(x, k, s, g, F.fftconv2d_bhl, 2e-2, tol64=5e-3)


def test_config5_full_launch_bf16_fwd_bwd():
    """Config 5 at full size: B=2, C=128, 64^3 bf16, radial filter sigma ~ U(2, 32)."""
    B, C, S = 2, 128, (64, 64, 64)
    assert _images_per_workgroup(B, C, S, S, adjoint=False) == 2
    assert _images_per_workgroup(B, C, S, S, adjoint=True) == 2
    gen = torch.Generator().manual_seed(0)
    x, k, s, g = _nd_full_case(B, C, S, S, torch.bfloat16, gen, sig=(2.0, 32.0))
    _check_nd_full(x, k, s, g, F.fftconv3d_bhl, 2e-2, tol64=5e-3)


def test_config3_full_launch_bf16_fwd_bwd():
    """Config 3 at full size (B=1, D=4096, L=262144, bf16 I/O, the benchmarked call pair
    through autograd): three sampled channels of y, gx, gk and gs against the oracle."""
    D, L = 4096, 262144
    c = causal1d_case_fast(1, D, L, torch.bfloat16, (1.0, 50.0), device="cuda", seed=5)
    xg = c.x.requires_grad_(True)
    kg = c.k[None].requires_grad_(True)
    sg = c.s.requires_grad_(True)
    y = F.causal_fftconv1d_bhl(xg, kg, sg)
    y.backward(c.g)
    torch.cuda.synchronize()
    ch = [0, 2049, D - 1]
    x = c.x.detach()[:, ch].cpu().requires_grad_(True)
    k = c.k.detach()[None, ch].cpu().requires_grad_(True)
    s = c.s.detach()[ch].cpu().requires_grad_(True)
    y_ref = causal_fftconv1d_torch(x, k, s)
    y_ref.backward(c.g[:, ch].cpu())
    assert y.dtype == torch.bfloat16
    assert rel_l2(y_ref, y[:, ch]) < 2e-2
    assert rel_l2(x.grad, xg.grad[:, ch]) < 2e-2
    assert rel_l2(k.grad, kg.grad[:, ch]) < 2e-2
    assert rel_l2(s.grad, sg.grad[ch]) < 2e-2
    y64 = causal_fftconv1d_np(x.detach().float().numpy(), k.detach()[0].numpy(), s.detach().float().numpy())
    assert rel_l2(y64, y[:, ch]) < 5e-3


def test_config2_full_launch_bf16():
    """Config 2 at full size (B=4, L=8192, 3*4096 channels, k=3 projection, k=128 mixer,
    skip = 0 as the config's formula), plus a fwd+bwd at the same size with an N(0,1)
    skip; four output channels (with their q, k, v input channels) against the oracle."""
    B, C, L = 4, 4096, 8192
    gen = torch.Generator(device="cuda").manual_seed(2)
    x = torch.randn(B, 3 * C, L, device="cuda", generator=gen).to(torch.bfloat16)
    wp = torch.randn(3 * C, 3, device="cuda", generator=gen)
    wm = torch.randn(C, 128, device="cuda", generator=gen) / 128 ** 0.5
    ch = _sampled(C)
    rows = ch + [C + c for c in ch] + [2 * C + c for c in ch]
    xs = x[:, rows].float().cpu()
    y = b2b_causal_conv1d(x, wp, wm, torch.zeros(C, device="cuda"))
    y_ref = b2b_causal_conv1d_torch(xs, wp[rows].cpu(), wm[ch].cpu(), torch.zeros(len(ch)))
    assert y.dtype == torch.bfloat16
    assert rel_l2(y_ref, y[:, ch].float()) < 2e-2
    del y
    sk = torch.randn(C, device="cuda", generator=gen)
    g = torch.randn(B, C, L, device="cuda", generator=gen).to(torch.bfloat16)
    xg, wpg, wmg, skg = (t.clone().requires_grad_(True) for t in (x, wp, wm, sk))
    y = b2b_causal_conv1d(xg, wpg, wmg, skg)
    y.backward(g)
    torch.cuda.synchronize()
    xr = xs.clone().requires_grad_(True)
    wpr = wp[rows].cpu().requires_grad_(True)
    wmr = wm[ch].cpu().requires_grad_(True)
    skr = sk[ch].cpu().requires_grad_(True)
    y_ref = b2b_causal_conv1d_torch(xr, wpr, wmr, skr)
    y_ref.float().backward(g[:, ch].float().cpu())
    assert rel_l2(y_ref, y[:, ch].float()) < 2e-2
    assert rel_l2(xr.grad, xg.grad[:, rows].float()) < 2e-2
    assert rel_l2(wpr.grad, wpg.grad[rows]) < 2e-2
    assert rel_l2(wmr.grad, wmg.grad[ch]) < 2e-2
    assert rel_l2(skr.grad, skg.grad[ch]) < 2e-2
