"""GPU tests of the channels-last -> channels-first layout change used by the BLH wrappers
(``nsq_batched_transpose``, :mod:`nvsubquadratic_amd.layout`): bitwise equal to torch's permute-copy for the
16-byte vector tiles and the element path (edge tiles, rows that are not 16-byte multiples), fp32 / bf16 /
fp16, and the gradient through a BLH wrapper equal to the same conv on a channels-first copy."""

import pytest
import torch

from nvsubquadratic_amd import fftconv_hip as F
from nvsubquadratic_amd.layout import channels_first_contiguous, transpose_inner_op

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,R,C", [(2, 128, 256), (1, 8192, 64), (3, 100, 72), (2, 67, 130), (1, 1, 9), (4, 64, 1)])
def test_transpose_matches_torch(dtype, B, R, C):
    print(f"transpose {dtype} B={B} R={R} C={C}", flush=True)
    x = torch.randn(B, R, C, device="cuda").to(dtype)
    y = transpose_inner_op(x)
    assert y.shape == (B, C, R) and y.is_contiguous()
    assert torch.equal(y, x.transpose(1, 2).contiguous())


@pytest.mark.parametrize("R", [65535 * 64 + 128, 65535 * 64 + 37])
def test_transpose_rows_beyond_65535_tiles(R):
    """More than 65535 row tiles (R > 65535 * 64, e.g. L = 2^22 on the 4-step plan): the row tiles sit on grid.x;
    a vector tile run and an element-path edge."""
    print(f"transpose long rows R={R}", flush=True)
    x = torch.randn(1, R, 8, device="cuda").to(torch.bfloat16)
    y = transpose_inner_op(x)
    assert torch.equal(y, x.transpose(1, 2).contiguous())
    v = x.movedim(-1, 1)  # the channels-last view a BLH wrapper hands over
    assert torch.equal(channels_first_contiguous(v), v.contiguous())


def test_channels_first_contiguous_views():
    x = torch.randn(2, 48, 40, 24, device="cuda").to(torch.bfloat16)  # BLH [B, X, Y, H]
    v = x.movedim(-1, 1)                                                # the rearranged view [B, H, X, Y]
    y = channels_first_contiguous(v)
    assert y.is_contiguous() and torch.equal(y, v.contiguous())
    z = torch.randn(2, 24, 48, 40, device="cuda")
    assert channels_first_contiguous(z) is z                            # already channels-first
    w = z[:, :, ::2]                                                    # another layout: Tensor.contiguous
    assert torch.equal(channels_first_contiguous(w), w.contiguous())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_blh_wrapper_gradients_equal_channels_first(dtype):
    """causal_fftconv1d_bhl_w_reshape on [B, L, H] against causal_fftconv1d_bhl on a channels-first copy, with a
    gradient that arrives channels-last: outputs and every gradient bitwise equal."""
    torch.manual_seed(0)
    B, L, H, K = 2, 4096, 48, 4096
    x = torch.randn(B, L, H, device="cuda").to(dtype).requires_grad_(True)
    k = (torch.randn(1, K, H, device="cuda") / 64).requires_grad_(True)
    s = torch.randn(H, device="cuda").to(dtype).requires_grad_(True)
    g = torch.randn(B, L, H, device="cuda").to(dtype)
    y = F.causal_fftconv1d_bhl_w_reshape(x, k, s)
    y.backward(g)
    x2 = x.detach().transpose(1, 2).contiguous().requires_grad_(True)
    k2 = k.detach().transpose(1, 2).contiguous().requires_grad_(True)
    s2 = s.detach().clone().requires_grad_(True)
    y2 = F.causal_fftconv1d_bhl(x2, k2, s2)
    y2.backward(g.transpose(1, 2).contiguous())
    assert torch.equal(y, y2.transpose(1, 2))
    assert torch.equal(x.grad, x2.grad.transpose(1, 2))
    assert torch.equal(k.grad, k2.grad.transpose(1, 2))
    assert torch.equal(s.grad, s2.grad)
