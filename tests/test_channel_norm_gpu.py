"""GPU parity of the gate + channel-RMSNorm + layout pass (nsq_channel_rmsnorm_fwd / _bwd through the C ABI) against
the CPU restatement of the reference's op sequence (oracle/norm_ref.py) and, at the config-4 Hyena shape, against
the same sequence in fp32 torch ops on the GPU."""

import pytest
import torch

from nvsubquadratic_amd import _lib
from nvsubquadratic_amd import norm_hip as N
from oracle.norm_ref import gated_channel_rmsnorm_ref

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-3}
ACT = {"identity": 0, "sigmoid": 1, "silu": 2}


def rel_l2(ref, out) -> float:
    ref, out = ref.detach().double().cpu(), out.detach().double().cpu()
    return float((out - ref).norm() / ref.norm().clamp_min(1e-30))


def _case(B, C, spatial, dtype, gate, channels_last, eps=1e-6, seed=0, gtol=None):
    print(f"case B={B} C={C} S={spatial} {dtype} gate={gate} channels_last={channels_last}", flush=True)
    g = torch.Generator().manual_seed(seed)
    y = torch.randn(B, C, *spatial, generator=g).to(dtype)
    v = torch.randn(B, C, *spatial, generator=g).to(dtype) if gate is not None else None
    w = (1 + 0.5 * torch.randn(C, generator=g)).float()
    dev = "cuda"
    yd = y.to(dev).requires_grad_()
    vd = v.to(dev).requires_grad_() if v is not None else None
    wd = w.to(dev).requires_grad_()
    out = N.gated_channel_rmsnorm(yd, vd, wd, eps, gate or "identity", channels_last_out=channels_last)
    gout = torch.randn(out.shape, generator=g).to(dtype)
    out.backward(gout.to(dev))
    torch.cuda.synchronize()
    yc = y.clone().requires_grad_()
    vc = v.clone().requires_grad_() if v is not None else None
    wc = w.clone().requires_grad_()
    ref = gated_channel_rmsnorm_ref(yc, vc, wc, eps, ACT[gate] if gate else 0, channels_last)
    ref.backward(gout)
    tol = TOL[dtype]
    gtol = gtol or tol
    assert out.shape == ref.shape and out.dtype == dtype
    assert rel_l2(ref, out) < tol
    assert rel_l2(yc.grad, yd.grad) < gtol
    if v is not None:
        assert rel_l2(vc.grad, vd.grad) < gtol
    assert rel_l2(wc.grad, wd.grad) < tol


@pytest.mark.parametrize("gate", [None, "sigmoid", "silu"])
@pytest.mark.parametrize("channels_last", [True, False])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_hyena_shape(gate, channels_last, dtype):
    _case(2, 384, (16, 16), dtype, gate, channels_last)


@pytest.mark.parametrize("B,C,spatial", [(3, 5, (33,)), (1, 1000, (7, 9)), (2, 3000, (10,)), (1, 1, (70,)), (2, 96, (104,)), (1, 3000, (16,)),
                                         (2, 257, (3, 5, 7))])
@pytest.mark.parametrize("channels_last", [True, False])
def test_ragged_shapes(B, C, spatial, channels_last):
    # One channel: xhat = +-1 up to eps, and the input gradient r dx (1 - xhat^2) cancels to a few fp32 ulps of dx in
    # the reference as well, so its gradients are compared at 1e-3.
    gtol = 1e-3 if C == 1 else None
    _case(B, C, spatial, torch.float32, "sigmoid", channels_last, gtol=gtol)
    _case(B, C, spatial, torch.bfloat16, "silu", channels_last, seed=1)


def test_several_tiles_per_workgroup_bf16():
    # C = 384 backward tiles hold 16 positions: 4 x 16384 positions = 4096 tiles over 512 workgroups (the
    # backward grid's cap), 8 tiles each
    _case(4, 384, (128, 128), torch.bfloat16, "sigmoid", True)


def test_channels_first_module_and_eps():
    torch.manual_seed(3)
    x = torch.randn(2, 96, 12, 12, device="cuda")
    m = N.HipRMSNormChannelFirst(96, eps=1e-3).cuda()
    with torch.no_grad():
        m.weight.copy_(torch.rand(96) + 0.5)
    out = m(x)
    ref = gated_channel_rmsnorm_ref(x.cpu(), None, m.weight.detach().cpu(), 1e-3, channels_last=False)
    assert rel_l2(ref, out) < 1e-5


def test_input_gradient_orthogonal_to_input_at_zero_eps():
    # scale invariance at eps = 0: sum_c dy_c y_c = 0 at every position (full cfg4 plane, fp32)
    torch.manual_seed(4)
    y = torch.randn(2, 384, 128, 128, device="cuda", requires_grad=True)
    w = torch.ones(384, device="cuda")
    out = N.gated_channel_rmsnorm(y, None, w, 0.0, channels_last_out=True)
    out.backward(torch.randn_like(out))
    dot = (y.grad * y.detach()).sum(1).abs()
    scale = (y.grad.norm(dim=1) * y.detach().norm(dim=1))
    assert float((dot / scale).max()) < 1e-5


def test_cfg4_shape_against_torch_fp32_sequence():
    # the Hyena output tail at config 4's shape (B=16, C=384, 128 x 128, bf16) against the reference's ops in fp32
    torch.manual_seed(5)
    B, C, S = 16, 384, (128, 128)
    y = torch.randn(B, C, *S, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    v = torch.randn(B, C, *S, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    w = (torch.rand(C, device="cuda") + 0.5).requires_grad_()
    out = N.hyena_output_norm(y, v, w, 1e-6, "sigmoid")
    gout = torch.randn_like(out)
    out.backward(gout)
    y32, v32 = y.detach().float().requires_grad_(), v.detach().float().requires_grad_()
    w32 = w.detach().clone().requires_grad_()
    u = (y32 * torch.sigmoid(v32)).movedim(1, -1)
    ref = w32 * (u * torch.rsqrt(u.pow(2).mean(-1, keepdim=True) + 1e-6))
    ref.backward(gout.float())
    assert out.shape == (B, *S, C)
    assert rel_l2(ref, out) < 2e-2
    assert rel_l2(y32.grad, y.grad) < 2e-2
    assert rel_l2(v32.grad, v.grad) < 2e-2
    assert rel_l2(w32.grad, w.grad) < 2e-2


def test_dw_deterministic():
    torch.manual_seed(6)
    y = torch.randn(4, 64, 4096, device="cuda", dtype=torch.bfloat16)
    v = torch.randn_like(y)
    w = torch.rand(64, device="cuda")
    g = torch.randn(4, 4096, 64, device="cuda", dtype=torch.bfloat16)
    r1 = N.gated_channel_rmsnorm_backward_op(g, y, v, w, 1e-6, 1, True)
    r2 = N.gated_channel_rmsnorm_backward_op(g, y, v, w, 1e-6, 1, True)
    for a, b in zip(r1, r2):
        assert torch.equal(a, b)


def test_argument_errors():
    y = torch.randn(1, 9000, 2, device="cuda")
    with pytest.raises(NotImplementedError, match="exceeds the LDS"):
        N.gated_channel_rmsnorm(y, None, torch.ones(9000, device="cuda"), channels_last_out=True)
    y = torch.randn(1, 4000, 2, device="cuda")
    with pytest.raises(NotImplementedError, match="exceeds the LDS"):
        N.gated_channel_rmsnorm_backward_op(y, y, None, torch.ones(4000, device="cuda"), 1e-6, 0, False)
    with pytest.raises(ValueError):
        N.gated_channel_rmsnorm(torch.randn(1, 4, 3, device="cuda"), None, torch.ones(5, device="cuda"))


def test_opcheck():
    y = torch.randn(2, 16, 24, device="cuda", requires_grad=True)
    v = torch.randn(2, 16, 24, device="cuda", requires_grad=True)
    w = torch.rand(16, device="cuda", requires_grad=True)
    torch.library.opcheck(N.gated_channel_rmsnorm_op, (y, v, w, 1e-6, 1, True))
    torch.library.opcheck(N.gated_channel_rmsnorm_op, (y, None, w, 1e-6, 0, False))
