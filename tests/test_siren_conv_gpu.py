"""GPU parity of the causal 1D conv whose SIREN filter is never formed (nsq_siren_fftconv1d_causal_*).

Checked against the CPU restatement of the reference chain (CKConvND's causal path, ckconv_nd.py:1149-1164 with
an identity mask): the SIREN network at the L causal points of the 2L - 1 grid (oracle/siren_ref.py), then the
causal FFT conv (oracle/fftconv_ref.py, fftconv.py:546-600), with autograd through both, on the same inputs.
Shapes take the 4-step plan (FFT lengths 2^15 .. 2^17 here): HD 16, 32 and 64, with and without biases and
shortcut, B = 1 .. 3.  Tolerances (fp32 I/O): output rel-L2 <= 2e-5, every gradient (x, shortcut, W_0, b_0, the
hidden weights and biases, W_out, b_out) <= 1e-4 -- the readout's gradient products run as bf16 three-product
splits (~2^-17 per product), as the unfused readout gradient does.  bf16 I/O at a longer shape against the unfused
HIP composition (siren_filter, then causal_fftconv1d_bhl).  Without forward state the backward recomputes the
transforms: bitwise equal to the state path; repeated calls are bitwise equal; shapes the fused plan runs take the
composition itself.
"""

import pytest
import torch

from nvsubquadratic_amd.fftconv_hip import causal_fftconv1d_bhl
from nvsubquadratic_amd.siren_hip import (HipSIRENKernelND, siren_causal_fftconv1d, siren_conv_fits, siren_filter,
                                          siren_grid)
from oracle.fftconv_ref import causal_fftconv1d_torch, rel_l2
from oracle.siren_ref import siren_mlp_torch, siren_params

pytestmark = pytest.mark.gpu

CASES = [  # (B, H, L, E, HD, nh, bias, shortcut)
    (2, 8, 8200, 32, 32, 2, True, True),
    (1, 16, 20000, 32, 16, 3, False, False),
    (2, 4, 9000, 32, 64, 1, True, True),
    (3, 6, 33000, 16, 32, 2, True, True),
]


def _setup(case, seed):
    B, H, L, E, HD, nh, bias, with_s = case
    grid = siren_grid((L,), (1.0,), (L,))[L - 1:].contiguous()  # [L, 1]: the points CKConvND's causal crop keeps
    params = siren_params(1, E, HD, nh, H, bias=bias, seed=seed)
    gen = torch.Generator().manual_seed(seed + 100)
    x = torch.randn(B, H, L, generator=gen)
    s = torch.randn(H, generator=gen) if with_s else None
    g = torch.randn(B, H, L, generator=gen)
    return grid, params, x, s, g


def _leaves(params, x, s):
    w0, b0, hw, hb, wo, bo = params
    return [w0, b0, *hw, *(hb or []), wo, bo, x, s]


def _split(ts, nh, bias):
    w0, b0 = ts[0], ts[1]
    hw = ts[2:2 + nh]
    hb = ts[2 + nh:2 + 2 * nh] if bias else None
    o = 2 + (2 * nh if bias else nh)
    return w0, b0, hw, hb, ts[o], ts[o + 1], ts[o + 2], ts[o + 3]


@pytest.mark.parametrize("case", CASES)
def test_matches_reference_chain(case):
    B, H, L, E, HD, nh, bias, with_s = case
    print(f"siren conv vs oracle chain {case}", flush=True)
    grid, params, x, s, g = _setup(case, 1)
    assert siren_conv_fits(B, H, L, L, HD)
    leaves = _leaves(params, x, s)
    ref = [None if t is None else t.clone().requires_grad_(True) for t in leaves]
    w0, b0, hw, hb, wo, bo, xr, sr = _split(ref, nh, bias)
    k = siren_mlp_torch(grid, w0, b0, hw, hb, wo, bo).t()  # [H, K]
    yr = causal_fftconv1d_torch(xr, k, sr)
    yr.backward(g)
    hip = [None if t is None else t.cuda().requires_grad_(True) for t in leaves]
    w0, b0, hw, hb, wo, bo, xh, sh = _split(hip, nh, bias)
    yh = siren_causal_fftconv1d(xh, grid.cuda(), w0, b0, hw, hb, wo, bo, sh)
    yh.backward(g.cuda())
    assert rel_l2(yr, yh) < 2e-5
    for r, h in zip(ref, hip):
        if r is not None:
            assert rel_l2(r.grad, h.grad) < 1e-4, r.shape


def _hip_run(case, seed, dtype=torch.float32):
    B, H, L, E, HD, nh, bias, with_s = case
    grid, params, x, s, g = _setup(case, seed)
    hip = [None if t is None else t.cuda().requires_grad_(True) for t in _leaves(params, x, s)]
    w0, b0, hw, hb, wo, bo, xh, sh = _split(hip, nh, bias)
    xd = xh.detach().to(dtype).requires_grad_(True)
    sd = None if sh is None else sh.detach().to(dtype).requires_grad_(True)
    y = siren_causal_fftconv1d(xd, grid.cuda(), w0, b0, hw, hb, wo, bo, sd)
    y.backward(g.cuda().to(dtype))
    grads = [t.grad for t in hip[:-2] if t is not None] + [xd.grad] + ([sd.grad] if sd is not None else [])
    return y.detach(), grads


def test_without_forward_state_is_bitwise_equal(monkeypatch):
    case = CASES[0]
    print(f"siren conv state / no state {case}", flush=True)
    y1, g1 = _hip_run(case, 2)
    monkeypatch.setenv("NSQ_STATE_MAX_BYTES", "0")  # the forward keeps nothing; the backward recomputes
    y0, g0 = _hip_run(case, 2)
    assert torch.equal(y1, y0)
    for a, b in zip(g1, g0):
        assert torch.equal(a, b)


def test_repeatable():
    case = CASES[3]
    print(f"siren conv repeat {case}", flush=True)
    ya, ga = _hip_run(case, 3)
    yb, gb = _hip_run(case, 3)
    assert torch.equal(ya, yb)
    for a, b in zip(ga, gb):
        assert torch.equal(a, b)


@pytest.mark.parametrize("B,H,L,dtype", [(2, 64, 65536, torch.bfloat16), (1, 32, 262144, torch.float16)])
def test_long_matches_unfused_composition(B, H, L, dtype):
    """The filter-free path against the HIP composition it replaces (filter formed, then the conv), 16-bit I/O."""
    print(f"siren conv vs composition B={B} H={H} L={L} {dtype}", flush=True)
    grid = siren_grid((L,), (1.0,), (L,))[L - 1:].contiguous().cuda()
    w0, b0, hw, hb, wo, bo = (None if t is None else (t.cuda() if isinstance(t, torch.Tensor) else
                                                      [u.cuda() for u in t]) for t in siren_params(1, 32, 32, 2, H,
                                                                                                   seed=6))
    gen = torch.Generator().manual_seed(9)
    x = torch.randn(B, H, L, generator=gen).to(dtype).cuda()
    s = torch.randn(H, generator=gen).to(dtype).cuda()
    g = torch.randn(B, H, L, generator=gen).to(dtype).cuda()

    def run(fused):
        leaves = [t.detach().clone().requires_grad_(True) for t in (w0, b0, *hw, *hb, wo, bo, x, s)]
        a, b_, h1, h2, c1, c2, o, ob, xx, ss = leaves
        if fused:
            y = siren_causal_fftconv1d(xx, grid, a, b_, [h1, h2], [c1, c2], o, ob, ss)
        else:
            y = causal_fftconv1d_bhl(xx, siren_filter(grid, a, b_, [h1, h2], [c1, c2], o, ob), ss)
        y.backward(g)
        return y.detach(), [t.grad for t in leaves]

    yf, gf = run(True)
    yu, gu = run(False)
    assert rel_l2(yu, yf) < 5e-3
    for i, (a, b) in enumerate(zip(gu, gf)):
        tol = 5e-3 if i >= len(gu) - 2 else 2e-4  # x and shortcut gradients are 16-bit
        assert rel_l2(a, b) < tol, i


def test_short_shapes_take_the_composition():
    B, H, L = 2, 8, 4000  # FFT length 8000 -> the fused plan, which reads the filter
    assert not siren_conv_fits(B, H, L, L, 32)
    grid = siren_grid((L,), (1.0,), (L,))[L - 1:].contiguous().cuda()
    w0, b0, hw, hb, wo, bo = siren_params(1, 32, 32, 2, H, seed=8)
    c = lambda t: t.cuda()  # noqa: E731
    x = torch.randn(B, H, L, generator=torch.Generator().manual_seed(1)).cuda()
    y = siren_causal_fftconv1d(x, grid, c(w0), c(b0), [c(w) for w in hw], [c(b) for b in hb], c(wo), c(bo))
    k = siren_filter(grid, c(w0), c(b0), [c(w) for w in hw], [c(b) for b in hb], c(wo), c(bo))
    assert torch.equal(y, causal_fftconv1d_bhl(x, k))


def test_module_causal_conv_matches_kernel_bhl():
    """HipSIRENKernelND.causal_fftconv1d equals the conv with its own causal filter (kernel_bhl)."""
    B, H, L = 2, 16, 12000
    print(f"siren module causal conv B={B} H={H} L={L}", flush=True)
    m = HipSIRENKernelND(out_dim=H, data_dim=1, mlp_hidden_dim=32, num_layers=3, embedding_dim=32, omega_0=10.0,
                         L_cache=L, use_bias=True).cuda()
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(B, H, L, generator=gen).cuda()
    s = torch.randn(H, generator=gen).cuda()
    g = torch.randn(B, H, L, generator=gen).cuda()
    y = m.causal_fftconv1d(x, s)
    y.backward(g)
    gm = [p.grad.clone() for p in m.parameters()]
    m.zero_grad()
    yr = causal_fftconv1d_bhl(x, m.kernel_bhl((L,), causal=True), s)
    yr.backward(g)
    assert rel_l2(yr, y) < 1e-5
    for a, p in zip(gm, m.parameters()):
        assert rel_l2(p.grad, a) < 1e-4


@pytest.mark.parametrize("B,H,L,K", [(1, 8, 20000, 5000), (2, 4, 12000, 12001)])
def test_filter_length_other_than_l(B, H, L, K):
    """K < L (a shorter filter grid) and K = L + 1, against the reference chain."""
    print(f"siren conv K != L B={B} H={H} L={L} K={K}", flush=True)
    grid = siren_grid((K,), (1.0,), (K,))[K - 1:].contiguous()  # K points
    w0, b0, hw, hb, wo, bo = siren_params(1, 32, 32, 2, H, seed=12)
    gen = torch.Generator().manual_seed(13)
    x = torch.randn(B, H, L, generator=gen)
    s = torch.randn(H, generator=gen)
    g = torch.randn(B, H, L, generator=gen)
    assert siren_conv_fits(B, H, L, K, 32)
    leaves = [w0, b0, *hw, *hb, wo, bo, x, s]
    ref = [t.clone().requires_grad_(True) for t in leaves]
    yr = causal_fftconv1d_torch(ref[8], siren_mlp_torch(grid, ref[0], ref[1], ref[2:4], ref[4:6], ref[6], ref[7]).t(),
                                ref[9])
    yr.backward(g)
    hip = [t.cuda().requires_grad_(True) for t in leaves]
    yh = siren_causal_fftconv1d(hip[8], grid.cuda(), hip[0], hip[1], hip[2:4], hip[4:6], hip[6], hip[7], hip[9])
    yh.backward(g.cuda())
    assert rel_l2(yr, yh) < 2e-5
    for r, h in zip(ref, hip):
        assert rel_l2(r.grad, h.grad) < 1e-4, r.shape
