"""GPU parity of the gate + channel-RMSNorm (and LayerNorm, L2) + layout pass (nsq_channel_*_fwd / _bwd through the C ABI) against
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


# --- QK-norm: L2 normalisation over channels (L2Norm, F.normalize) ----------------------------------------------
def _l2_case(B, C, spatial, dtype, channels_last, eps=1e-12, seed=0, tiny=False):
    from oracle.norm_ref import l2norm_ref

    print(f"l2 case B={B} C={C} S={spatial} {dtype} channels_last={channels_last} eps={eps}", flush=True)
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, C, *spatial, generator=g)
    if tiny:  # every other position far below eps: the clamped branch
        x[..., ::2] *= 1e-6
    x = x.to(dtype)
    xd = x.cuda().requires_grad_()
    out = N.channel_l2norm(xd, eps, channels_last_out=channels_last)
    gout = torch.randn(out.shape, generator=g).to(dtype)
    out.backward(gout.cuda())
    x64 = x.double().requires_grad_()
    ref = l2norm_ref(x64, 1, eps)
    ref = ref.movedim(1, -1) if channels_last else ref
    ref.backward(gout.double())
    assert out.shape == ref.shape and out.dtype == dtype
    tol = {torch.float32: 1e-6, torch.bfloat16: 5e-3, torch.float16: 1e-3}[dtype]
    assert rel_l2(ref, out) < tol
    if C == 1:  # out = sign(x): the exact input gradient is zero; the kernel's is rounding noise of dout / |x|
        scale = float((gout.double() / x64.detach().reshape(gout.shape) if not channels_last else
                       gout.double() / x64.detach().movedim(1, -1)).abs().max())
        assert float(xd.grad.double().cpu().abs().max()) < 10 * tol * scale
    else:
        assert rel_l2(x64.grad, xd.grad) < tol * 4
    if dtype != torch.float32:  # the same dtype's restatement (its norm rounded as torch rounds it)
        xr = x.clone().requires_grad_()
        r2 = l2norm_ref(xr, 1, eps)
        r2 = r2.movedim(1, -1) if channels_last else r2
        assert rel_l2(r2.float(), out.float()) < tol


@pytest.mark.parametrize("channels_last", [True, False])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,C,spatial", [(2, 384, (16, 16)), (3, 5, (7, 9)), (1, 257, (33,)), (2, 1000, (3, 5)),
                                         (1, 1, (64,)), (4, 64, (128, 128))])
def test_l2norm_over_channels(B, C, spatial, dtype, channels_last):
    _l2_case(B, C, spatial, dtype, channels_last)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_l2norm_clamped_positions(dtype):
    # eps 1e-3 against norms of ~1e-5 at every other position: out = x / eps there, dx = dout / eps
    _l2_case(2, 48, (8, 10), dtype, False, eps=1e-3, tiny=True)


def test_hip_l2norm_module_layouts():
    """HipL2Norm (L2Norm's interface): dim=1 on [B, C, *S]; dim=-1 on a channels-first tensor viewed channels-last
    (the Hyena operator's movedim) and on a contiguous channels-last tensor; all equal torch's F.normalize."""
    torch.manual_seed(1)
    x = torch.randn(2, 96, 12, 10, device="cuda")
    m1, m2 = N.HipL2Norm(dim=1), N.HipL2Norm()
    assert m1.channels_first and not m2.channels_first
    ref = torch.nn.functional.normalize(x, dim=1)
    assert rel_l2(ref, m1(x)) < 1e-6
    v = x.movedim(1, -1)
    out = m2(v)
    assert out.shape == v.shape and rel_l2(torch.nn.functional.normalize(v, dim=-1), out) < 1e-6
    c = v.contiguous()
    assert rel_l2(torch.nn.functional.normalize(c, dim=-1), m2(c)) < 1e-6
    with pytest.raises(NotImplementedError):
        N.HipL2Norm(dim=2)(x)


def test_l2norm_opcheck():
    x = torch.randn(2, 40, 33, device="cuda", requires_grad=True)
    torch.library.opcheck(N.channel_l2norm_op, (x, 1e-12, True))
    torch.library.opcheck(N.channel_l2norm_op, (x, 1e-12, False))


# --- LayerNorm over channels (torch.nn.LayerNorm(C) at the pixelhyena_norm site) ---------------------------------
def _ln_case(B, C, spatial, dtype, gate, channels_last, affine=True, use_bias=True, eps=1e-5, seed=0, gtol=None):
    from oracle.norm_ref import gated_channel_layernorm_ref

    print(f"ln case B={B} C={C} S={spatial} {dtype} gate={gate} channels_last={channels_last} affine={affine} "
          f"bias={use_bias}", flush=True)
    g = torch.Generator().manual_seed(seed)
    y = (0.7 * torch.randn(B, C, *spatial, generator=g) + 0.3).to(dtype)  # a nonzero mean per position
    v = torch.randn(B, C, *spatial, generator=g).to(dtype) if gate is not None else None
    w = (1 + 0.5 * torch.randn(C, generator=g)).float() if affine else None
    b = (0.2 * torch.randn(C, generator=g)).float() if affine and use_bias else None
    dev = "cuda"
    leaves = [t.to(dev).requires_grad_() if t is not None else None for t in (y, v, w, b)]
    out = N.gated_channel_layernorm(*leaves, eps, gate or "identity", channels_last_out=channels_last)
    gout = torch.randn(out.shape, generator=g).to(dtype)
    out.backward(gout.to(dev))
    torch.cuda.synchronize()
    refs = [t.clone().requires_grad_() if t is not None else None for t in (y, v, w, b)]
    ref = gated_channel_layernorm_ref(*refs, eps, ACT[gate] if gate else 0, channels_last)
    ref.backward(gout)
    tol = TOL[dtype]
    gtol = gtol or tol
    assert out.shape == ref.shape and out.dtype == dtype
    assert rel_l2(ref, out) < tol
    for r, d in zip(refs, leaves):
        if r is not None:
            assert rel_l2(r.grad, d.grad) < (tol if r.dtype == torch.float32 and r.dim() == 1 else gtol)


@pytest.mark.parametrize("gate", [None, "silu"])
@pytest.mark.parametrize("channels_last", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_layernorm_hyena_shape(gate, channels_last, dtype):
    _ln_case(2, 384, (32, 32), dtype, gate, channels_last)


@pytest.mark.parametrize("B,C,spatial,affine,use_bias", [(3, 40, (7, 5), True, True), (1, 257, (33,), True, False),
                                                          (2, 64, (3, 3, 3), False, False), (2, 3, (100,), True, True)])
def test_layernorm_ragged_shapes_and_affine(B, C, spatial, affine, use_bias):
    _ln_case(B, C, spatial, torch.float32, "sigmoid", False, affine=affine, use_bias=use_bias, seed=1)


def test_layernorm_module_drop_in():
    """HipLayerNormChannels on [B, C, *S] equals torch.nn.LayerNorm(C) on the channels-last view."""
    torch.manual_seed(7)
    ref = torch.nn.LayerNorm(48).cuda()
    with torch.no_grad():
        ref.weight.copy_(1 + 0.3 * torch.randn(48))
        ref.bias.copy_(0.1 * torch.randn(48))
    mod = N.HipLayerNormChannels(48).cuda()
    mod.load_state_dict(ref.state_dict())
    assert mod.channels_first
    x = torch.randn(2, 48, 9, 11, device="cuda", requires_grad=True)
    xr = x.detach().clone().requires_grad_()
    y = mod(x)
    yr = ref(xr.movedim(1, -1)).movedim(-1, 1)
    g = torch.randn_like(y)
    y.backward(g)
    yr.backward(g)
    assert rel_l2(yr, y) < 1e-5
    assert rel_l2(xr.grad, x.grad) < 1e-5
    assert rel_l2(ref.weight.grad, mod.weight.grad) < 1e-5
    assert rel_l2(ref.bias.grad, mod.bias.grad) < 1e-5


def test_layernorm_gradients_deterministic_and_limits():
    torch.manual_seed(8)
    y = torch.randn(4, 64, 4096, device="cuda", dtype=torch.bfloat16)
    w = torch.rand(64, device="cuda")
    g = torch.randn(4, 64, 4096, device="cuda", dtype=torch.bfloat16)
    r1 = N.gated_channel_layernorm_backward_op(g, y, None, w, True, 1e-5, 0, False)
    r2 = N.gated_channel_layernorm_backward_op(g, y, None, w, True, 1e-5, 0, False)
    for a, b in zip(r1, r2):
        assert torch.equal(a, b)
    lib = _lib.get_lib()
    assert lib.nsq_channel_layernorm_bwd_workspace_bytes(1, 3241, 8) > 0
    assert lib.nsq_channel_layernorm_bwd_workspace_bytes(1, 3242, 8) == 0
    yb = torch.randn(1, 3300, 2, device="cuda", requires_grad=True)
    with pytest.raises(NotImplementedError, match="C <= 3241"):
        N.gated_channel_layernorm(yb, None, torch.ones(3300, device="cuda"), None)


def test_layernorm_opcheck():
    y = torch.randn(2, 16, 24, device="cuda", requires_grad=True)
    v = torch.randn(2, 16, 24, device="cuda", requires_grad=True)
    w = torch.rand(16, device="cuda", requires_grad=True)
    b = torch.rand(16, device="cuda", requires_grad=True)
    torch.library.opcheck(N.gated_channel_layernorm_op, (y, v, w, b, 1e-5, 2, True))
    torch.library.opcheck(N.gated_channel_layernorm_op, (y, None, None, None, 1e-5, 0, False))


# GroupNorm over channels, channels-first (the pixelhyena_norm site with torch.nn.GroupNorm(G, C))

def _gn_case(B, C, spatial, G, dtype, gate, affine=True, eps=1e-5, seed=0, offset=0.3, tol=None, gtol=None):
    from oracle.norm_ref import gated_channel_groupnorm_ref

    print(f"gn case B={B} C={C} S={spatial} G={G} {dtype} gate={gate} affine={affine}", flush=True)
    g = torch.Generator().manual_seed(seed)
    y = (0.7 * torch.randn(B, C, *spatial, generator=g) + offset).to(dtype)
    v = torch.randn(B, C, *spatial, generator=g).to(dtype) if gate is not None else None
    w = (1 + 0.5 * torch.randn(C, generator=g)).float() if affine else None
    b = (0.2 * torch.randn(C, generator=g)).float() if affine else None
    dev = "cuda"
    leaves = [t.to(dev).requires_grad_() if t is not None else None for t in (y, v, w, b)]
    out = N.gated_channel_groupnorm(*leaves, G, eps, gate or "identity")
    gout = torch.randn(out.shape, generator=g).to(dtype)
    out.backward(gout.to(dev))
    torch.cuda.synchronize()
    refs = [t.clone().requires_grad_() if t is not None else None for t in (y, v, w, b)]
    ref = gated_channel_groupnorm_ref(*refs, G, eps, ACT[gate] if gate else 0)
    ref.backward(gout)
    tol = tol or TOL[dtype]
    gtol = gtol or tol
    assert out.shape == ref.shape and out.dtype == dtype
    assert rel_l2(ref, out) < tol
    for r, d in zip(refs, leaves):
        if r is not None:
            assert rel_l2(r.grad, d.grad) < (tol if r.dtype == torch.float32 and r.dim() == 1 else gtol)


@pytest.mark.parametrize("gate", [None, "sigmoid"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_groupnorm_hyena_shape(gate, dtype):
    # the reference's configs: GroupNorm(num_groups=1, C) on [B, C, H, W]
    _gn_case(2, 384, (32, 32), 1, dtype, gate)


@pytest.mark.parametrize("B,C,spatial,G,affine", [(3, 12, (7, 5), 4, True), (2, 8, (33,), 8, True),
                                                   (1, 1, (70,), 1, False), (2, 6, (1,), 3, True),
                                                   (2, 16, (3, 4, 5), 2, True), (1, 4, (100003,), 1, True),
                                                   (2, 32, (64, 64), 1, False)])
def test_groupnorm_ragged_shapes_and_groups(B, C, spatial, G, affine):
    _gn_case(B, C, spatial, G, torch.float32, "silu", affine=affine, seed=1)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_groupnorm_ragged_16bit(dtype):
    # S not a multiple of the 8-wide vectors: the scalar passes
    _gn_case(2, 24, (13, 7), 3, dtype, "silu", seed=2)


def test_groupnorm_large_mean():
    # A mean 1400x the spread (fp32 in and out).  torch's scale / shift form u a + (b - mean a) rounds two terms of
    # size mean / std to fp32, so outputs of unit size carry errors near 1e-4 in any fp32 implementation of it
    # (1 ulp of a or of mean moves them that much): 5e-4 is that bound.  E[u^2] - E[u]^2 in fp32 would lose the
    # variance outright (an error of about 10% here); the shifted row sums keep it.
    _gn_case(2, 16, (40, 40), 2, torch.float32, None, offset=1000.0, seed=3, tol=5e-4, gtol=5e-4)


def test_groupnorm_misaligned_pointers():
    # inputs at an offset of one element: the scalar passes on unaligned rows
    from oracle.norm_ref import gated_channel_groupnorm_ref

    B, C, S, G = 2, 8, 64, 2
    base = torch.randn(B * C * S + 1, device="cuda").to(torch.bfloat16)
    y = base[1:].view(B, C, S)
    w = torch.rand(C, device="cuda") + 0.5
    out, mean, rstd = N.gated_channel_groupnorm_op(y, None, w, None, G, 1e-5, 0)
    ref = gated_channel_groupnorm_ref(y.cpu(), None, w.cpu(), None, G, 1e-5, 0)
    assert rel_l2(ref, out) < TOL[torch.bfloat16]
    xg = y.double().reshape(B, G, -1)
    assert torch.allclose(mean.double(), xg.mean(-1), rtol=1e-5, atol=1e-5)
    assert torch.allclose(rstd.double(), torch.rsqrt(xg.var(-1, unbiased=False) + 1e-5), rtol=1e-4)


def test_groupnorm_module_drop_in():
    """HipGroupNorm equals torch.nn.GroupNorm on [B, C, *S], outputs and every gradient."""
    torch.manual_seed(9)
    for G in (1, 4):
        ref = torch.nn.GroupNorm(G, 48).cuda()
        with torch.no_grad():
            ref.weight.copy_(1 + 0.3 * torch.randn(48))
            ref.bias.copy_(0.1 * torch.randn(48))
        mod = N.HipGroupNorm(G, 48).cuda()
        mod.load_state_dict(ref.state_dict())
        assert mod.channels_first
        x = torch.randn(2, 48, 9, 11, device="cuda", requires_grad=True)
        xr = x.detach().clone().requires_grad_()
        y = mod(x)
        yr = ref(xr)
        gr = torch.randn_like(y)
        y.backward(gr)
        yr.backward(gr)
        assert rel_l2(yr, y) < 1e-5
        assert rel_l2(xr.grad, x.grad) < 1e-5
        assert rel_l2(ref.weight.grad, mod.weight.grad) < 1e-5
        assert rel_l2(ref.bias.grad, mod.bias.grad) < 1e-5


def test_groupnorm_gradients_deterministic():
    torch.manual_seed(10)
    y = torch.randn(4, 64, 4096, device="cuda", dtype=torch.bfloat16)
    w = torch.rand(64, device="cuda")
    g = torch.randn(4, 64, 4096, device="cuda", dtype=torch.bfloat16)
    _, mean, rstd = N.gated_channel_groupnorm_op(y, None, w, None, 1, 1e-5, 0)
    r1 = N.gated_channel_groupnorm_backward_op(g, y, None, w, mean, rstd, True, 0)
    r2 = N.gated_channel_groupnorm_backward_op(g, y, None, w, mean, rstd, True, 0)
    for a, b in zip(r1, r2):
        assert torch.equal(a, b)


def test_groupnorm_argument_errors():
    y = torch.randn(2, 6, 8, device="cuda")
    with pytest.raises(ValueError, match="divisible"):
        N.gated_channel_groupnorm(y, None, None, None, 4)
    with pytest.raises(ValueError, match="channel_groupnorm_fwd: num_channels 6 must be divisible"):
        N.gated_channel_groupnorm_op(y, None, None, None, 4, 1e-5, 0)  # the library's own check
    lib = _lib.get_lib()
    assert lib.nsq_channel_groupnorm_workspace_bytes(2, 6, 4, _lib.NSQ_DIR_FWD) == 0
    assert lib.nsq_channel_groupnorm_workspace_bytes(2, 6, 3, _lib.NSQ_DIR_FWD) == 2 * 6 * 8
    assert lib.nsq_channel_groupnorm_workspace_bytes(2, 6, 3, _lib.NSQ_DIR_BWD) == 2 * 6 * 8 + 2 * 3 * 8


def test_groupnorm_opcheck():
    y = torch.randn(2, 16, 24, device="cuda", requires_grad=True)
    v = torch.randn(2, 16, 24, device="cuda", requires_grad=True)
    w = torch.rand(16, device="cuda", requires_grad=True)
    b = torch.rand(16, device="cuda", requires_grad=True)
    torch.library.opcheck(N.gated_channel_groupnorm_op, (y, v, w, b, 4, 1e-5, 2))
    torch.library.opcheck(N.gated_channel_groupnorm_op, (y, None, None, None, 1, 1e-5, 0))
