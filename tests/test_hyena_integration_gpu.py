"""Hyena-level integration of the hip backend (GPU).

Composes the Hyena operator's data path (nvsubquadratic/modules/hyena_nd.py:498-583:
BLH -> BHL, short conv on [Q; K; V], split, gate z = Q * sigmoid(K), global conv
with shortcut via the CKConvND BHL entry point (ckconv_nd.py:1054-1062),
y * sigmoid(V), BHL -> BLH) once with the hip backend (HipCausalConv1d +
dispatch.hip_fftconv_fns) and once with the CPU oracle functions, for 1D causal,
2D and 3D, forward and backward.  The norms and the implicit-kernel generator of
the reference are out of the hot path; the kernel is a given fp32 tensor here.
"""

import pytest
import torch
from einops import rearrange

from nvsubquadratic_amd.dispatch import hip_fftconv_fns
from nvsubquadratic_amd.modules import HipCausalConv1d
from oracle.direct_ref import causal_conv1d_torch
from oracle.fftconv_ref import causal_fftconv1d_torch, fftconv_nd_torch, rel_l2


pytestmark = pytest.mark.gpu


def _hyena(q, k, v, short_conv, fft_bhl, kernel, shortcut):
    q, k, v = (rearrange(t, "b ... c -> b c ...") for t in (q, k, v))
    C = q.shape[1]
    if short_conv is not None:
        x = short_conv(torch.cat([q, k, v], dim=1))
        q, k, v = (t.contiguous() for t in x.split(C, dim=1))
    z = q * torch.sigmoid(k)
    y = fft_bhl(z, kernel, shortcut)
    y = y * torch.sigmoid(v)
    return rearrange(y, "b c ... -> b ... c")


@pytest.mark.parametrize("data_dim,spatial,kshape", [(1, (512,), (512,)), (2, (16, 16), (31, 31)), (3, (8, 8, 8), (15, 15, 15))])
def test_hyena_block_hip_vs_oracle(data_dim, spatial, kshape):
    torch.manual_seed(0)
    B, C = 2, 12
    q, k, v = (torch.randn(B, *spatial, C, requires_grad=True) for _ in range(3))
    kernel = torch.randn(1, C, *kshape, requires_grad=True)
    shortcut = torch.randn(C, requires_grad=True)
    _, fft_bhl = hip_fftconv_fns(data_dim, is_causal=(data_dim == 1))
    short = None
    w_short = torch.randn(3 * C, 3)
    if data_dim == 1:
        short = HipCausalConv1d(3 * C, 3 * C, 3, groups=3 * C).cuda()
        with torch.no_grad():
            short.weight.copy_(w_short.unsqueeze(1))

    # oracle composition on the CPU
    ref_short = (lambda x: causal_conv1d_torch(x, w_short)) if data_dim == 1 else None
    ref_fft = causal_fftconv1d_torch if data_dim == 1 else fftconv_nd_torch
    y_ref = _hyena(q, k, v, ref_short, ref_fft, kernel, shortcut)
    g = torch.randn_like(y_ref)
    y_ref.backward(g)

    args = [t.detach().cuda().requires_grad_(True) for t in (q, k, v, kernel, shortcut)]
    y = _hyena(args[0], args[1], args[2], short, fft_bhl, args[3], args[4])
    y.backward(g.cuda())
    assert rel_l2(y_ref, y) < 1e-4
    for ref_t, hip_t in zip((q, k, v, kernel, shortcut), args):
        assert rel_l2(ref_t.grad, hip_t.grad) < 1e-4


@pytest.mark.parametrize("data_dim,spatial,kshape,fft_padding",
                         [(1, (256,), (256,), "circular"), (2, (32, 16), (32, 16), "circular"),
                          (2, (32, 16), (63, 16), ["zero", "circular"]),
                          (3, (16, 16, 16), (16, 31, 16), ["circular", "zero", "circular"])])
def test_hyena_block_periodic_boundaries(data_dim, spatial, kshape, fft_padding):
    """The Well-style configs: fft_padding="circular" (grid_type "single": K = S) and per-axis lists."""
    from oracle.circular_ref import mixed_fftconv_torch
    from nvsubquadratic_amd.dispatch import resolve_periodic

    torch.manual_seed(1)
    B, C = 2, 8
    q, k, v = (torch.randn(B, *spatial, C, requires_grad=True) for _ in range(3))
    kernel = torch.randn(1, C, *kshape, requires_grad=True)
    shortcut = torch.randn(C, requires_grad=True)
    _, fft_bhl = hip_fftconv_fns(data_dim, False, fft_padding)
    periodic = resolve_periodic(fft_padding, data_dim)
    y_ref = _hyena(q, k, v, None, lambda x, kk, s: mixed_fftconv_torch(x, kk, periodic, s, torch.float64),
                   kernel, shortcut)
    g = torch.randn_like(y_ref)
    y_ref.backward(g)
    args = [t.detach().cuda().requires_grad_(True) for t in (q, k, v, kernel, shortcut)]
    y = _hyena(args[0], args[1], args[2], None, fft_bhl, args[3], args[4])
    y.backward(g.cuda())
    assert rel_l2(y_ref, y) < 1e-4
    for ref_t, hip_t in zip((q, k, v, kernel, shortcut), args):
        assert rel_l2(ref_t.grad, hip_t.grad) < 1e-4
