"""GPU parity of the one-kernel 2D forward (csrc/fftconv2d_image.h).

A forward that keeps no state for a backward (no-grad inference, the config-4
benchmark step) runs whole images in one kernel when the FFT plane is 256 x 256
(zero-padded axes, S0 and S2 <= 128, shared filter, no gates).  Its column DFTs
are split into even and odd 128-point halves, so its rounding differs from the
three-pass plan's; both are checked against the float32 oracle (the reference's
torch.fft path, ops/fftconv.py:662-733) and against each other.  The three-pass
plan runs the same call when a backward-sized workspace is given (the forward
then keeps its state), which is how these tests reach both.

Tolerances: rel-L2 <= 1e-4 fp32 and <= 2e-2 bf16/fp16 I/O against the oracle;
image path against three-pass path <= 1e-5 (fp32) and <= 5e-3 (16-bit outputs,
last-bit rounding flips).
"""

import pytest
import torch

from nvsubquadratic_amd import _lib
from nvsubquadratic_amd import fftconv_hip as F
from nvsubquadratic_amd.workloads import radial_filter
from oracle.fftconv_ref import fftconv_nd_np, fftconv_nd_torch, rel_l2


pytestmark = pytest.mark.gpu


def _bwd_workspace(x, k):
    """A backward-sized workspace: the forward keeps its state and runs the three-pass plan."""
    lib = _lib.get_lib()
    B, H = x.shape[:2]
    need = lib.nsq_fftconv_nd_workspace_bytes(2, B, H, _lib.i64_array(x.shape[2:]), _lib.i64_array(k.shape[1:]), 1,
                                              _lib.NSQ_DIR_BWD)
    return torch.empty(need, dtype=torch.uint8, device=x.device)


def _both_paths(x, k, s):
    y_img = torch.empty_like(x)
    F.fftconv_nd_fwd_raw(x, k, s, y_img, 1)
    y_3p = torch.empty_like(x)
    F.fftconv_nd_fwd_raw(x, k, s, y_3p, 1, _bwd_workspace(x, k))
    torch.cuda.synchronize()
    return y_img, y_3p


CASES = [
    # (B, H, S, K, dtype, shortcut)
    (2, 8, (128, 128), (128, 128), torch.float32, True),    # config 4's image and filter
    (3, 16, (128, 128), (128, 128), torch.bfloat16, True),
    (2, 5, (100, 96), (64, 96), torch.float32, False),      # H not a multiple of 8, S0 != S2
    (1, 16, (128, 128), (4, 4), torch.float16, True),       # short filter: crop offset 2
    (2, 8, (120, 128), (17, 252), torch.bfloat16, True),    # K2 near 2 S2: crop offset 126
    (2, 8, (65, 72), (130, 120), torch.float32, True),      # K0 > S0: crop offset 65
]


@pytest.mark.parametrize("B,H,S,K,dtype,has_s", CASES)
def test_image_forward_matches_oracle_and_three_pass(B, H, S, K, dtype, has_s):
    print(f"image fwd B={B} H={H} S={S} K={K} {dtype} shortcut={has_s}", flush=True)
    torch.manual_seed(7)
    x = torch.randn(B, H, *S).to(dtype)
    k = torch.randn(H, *K) / (K[0] * K[1]) ** 0.5
    s = torch.randn(H).to(dtype) if has_s else None
    y_ref = fftconv_nd_torch(x, k[None], s)
    xg, kg, sg = x.cuda(), k.cuda(), (s.cuda() if has_s else None)
    y_img, y_3p = _both_paths(xg, kg, sg)
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    assert rel_l2(y_ref, y_img) < tol
    assert rel_l2(y_3p, y_img) < (1e-5 if dtype == torch.float32 else 5e-3)
    if dtype == torch.float32:
        # a different summation order: the image kernel, not the three-pass plan, produced y_img
        assert not torch.equal(y_img, y_3p)
        y64 = fftconv_nd_np(x.double().numpy(), k[None].double().numpy(), s.double().numpy() if has_s else None)
        assert rel_l2(y64, y_img) < 1e-5
    # the op (no grad) takes the same path
    with torch.no_grad():
        y_op = F.fftconv2d_bhl(xg, kg[None], sg)
    assert torch.equal(y_op, y_img)


def test_image_forward_full_config4_launch():
    """Config 4 at full size (B=16, C=384, 128^2, bf16): sampled channels against the oracle, all
    channels against the three-pass plan."""
    B, C, S = 16, 384, 128
    gen = torch.Generator().manual_seed(0)
    x = torch.randn(B, C, S, S, generator=gen).to(torch.bfloat16)
    k = radial_filter(C, S, 4.0, 64.0, 2, gen)
    s = torch.randn(C, generator=gen).to(torch.bfloat16)
    print("image fwd config 4 full launch", flush=True)
    xg, kg, sg = x.cuda(), k.cuda(), s.cuda()
    y_img, y_3p = _both_paths(xg, kg, sg)
    assert rel_l2(y_3p.float(), y_img.float()) < 5e-3
    for h in sorted({0, 1, C // 2 + 1, C - 1}):
        y_ref = fftconv_nd_torch(x[:, h:h + 1], k[h:h + 1][None], s[h:h + 1])
        assert rel_l2(y_ref, y_img[:, h:h + 1]) < 2e-2
        y64 = fftconv_nd_np(x[:, h:h + 1].double().numpy(), k[h:h + 1][None].double().numpy(),
                            s[h:h + 1].double().numpy())
        assert rel_l2(y64, y_img[:, h:h + 1]) < 5e-3


def test_image_forward_not_taken_with_state_or_gradients():
    """With a gradient wanted the forward keeps its state for the backward (three-pass plan), and
    the results of the two paths agree to fp32 rounding."""
    torch.manual_seed(3)
    x = torch.randn(2, 8, 128, 128, device="cuda", requires_grad=True)
    k = torch.randn(1, 8, 128, 128, device="cuda", requires_grad=True)
    y_grad = F.fftconv2d_bhl(x, k)
    with torch.no_grad():
        y_inf = F.fftconv2d_bhl(x, k)
    assert rel_l2(y_grad.detach(), y_inf) < 1e-5
    y_grad.sum().backward()
    assert torch.isfinite(x.grad).all() and torch.isfinite(k.grad).all()
