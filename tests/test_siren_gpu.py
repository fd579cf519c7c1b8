"""GPU parity of the HIP SIREN filter generation against the CPU restatement (oracle/siren_ref.py).

The reference network (kernels_nd.py:876-1190 without FiLM) at the shapes its configs use (embedding and
hidden width 32, 3 layers, 160-384 channels; examples/vit5_imagenet: KERNEL_* settings) and the long 1D
grid of a Hyena layer (4096 channels).  Forward: rel-L2 <= 1e-5 against float64 and float32 evaluations.
Backward: every weight and bias gradient against the restatement's autograd (float64), rel-L2 <= 1e-4;
repeated backward calls are bitwise equal (fixed-order reductions).
"""

import pytest
import torch

from nvsubquadratic_amd.siren_hip import HipSIRENKernelND, siren_filter, siren_grid
from oracle.fftconv_ref import rel_l2
from oracle.siren_ref import siren_mlp_torch, siren_params


pytestmark = pytest.mark.gpu

CASES = [  # (d, grid shape, E, HD, nh, H, bias)
    (1, (599,), 32, 32, 2, 160, True),
    (2, (27, 27), 32, 32, 2, 384, True),
    (3, (9, 7, 5), 16, 64, 1, 64, False),
    (1, (4095,), 64, 16, 3, 256, True),
    (2, (13, 11), 128, 128, 3, 32, True),
    (1, (16383,), 32, 32, 2, 4096, True),
]


def _grid(shape):
    return siren_grid([(s + 1) // 2 + 3 for s in shape], [1.0] * len(shape), [(s + 1) // 2 for s in shape])


def _run(case, seed=0):
    d, shape, E, HD, nh, H, bias = case
    grid = _grid(shape).reshape(-1, d)
    params = siren_params(d, E, HD, nh, H, bias=bias, seed=seed)
    return grid, params


@pytest.mark.parametrize("case", CASES)
def test_forward_matches_restatement(case):
    grid, (w0, b0, hw, hb, wo, bo) = _run(case)
    print(f"siren fwd {case}", flush=True)
    dev = lambda t: None if t is None else t.cuda()  # noqa: E731
    k = siren_filter(grid.cuda(), dev(w0), dev(b0), [w.cuda() for w in hw], None if hb is None else
                     [b.cuda() for b in hb], dev(wo), dev(bo))
    assert k.shape == (wo.shape[0], grid.shape[0]) and k.dtype == torch.float32
    ref64 = siren_mlp_torch(grid, w0, b0, hw, hb, wo, bo, dtype=torch.float64).t()
    ref32 = siren_mlp_torch(grid, w0, b0, hw, hb, wo, bo).t()
    assert rel_l2(ref64, k) < 1e-5
    assert rel_l2(ref32, k) < 1e-5


# the last case is long enough for the readout's split weight-gradient product (16 slices + a remainder)
BWD_CASES = CASES[:5] + [(1, (131071,), 32, 32, 2, 64, True)]


@pytest.mark.parametrize("case", BWD_CASES)
def test_backward_matches_restatement(case):
    grid, (w0, b0, hw, hb, wo, bo) = _run(case, seed=1)
    print(f"siren bwd {case}", flush=True)
    leaves = [w0, b0, *hw, *(hb or []), wo, bo]
    ref = [None if t is None else t.double().requires_grad_(True) for t in leaves]
    nh = len(hw)

    def split(ts):
        w0_, b0_ = ts[0], ts[1]
        hw_ = ts[2:2 + nh]
        hb_ = ts[2 + nh:2 + 2 * nh] if hb is not None else None
        return w0_, b0_, hw_, hb_, ts[-2], ts[-1]

    y = siren_mlp_torch(grid.double(), *split(ref), dtype=torch.float64)
    g = torch.randn(y.shape, dtype=torch.float64, generator=torch.Generator().manual_seed(5))
    y.backward(g)
    hip = [None if t is None else t.cuda().requires_grad_(True) for t in leaves]
    w0_, b0_, hw_, hb_, wo_, bo_ = split(hip)
    k = siren_filter(grid.cuda(), w0_, b0_, hw_, hb_, wo_, bo_)
    k.backward(g.t().float().cuda())
    for r, h in zip(ref, hip):
        if r is None:
            continue
        assert rel_l2(r.grad, h.grad) < 1e-4
    first = [None if t is None else t.grad.clone() for t in hip]
    for t in hip:
        if t is not None:
            t.grad = None
    siren_filter(grid.cuda(), w0_, b0_, hw_, hb_, wo_, bo_).backward(g.t().float().cuda())
    for a, t in zip(first, hip):
        if t is not None:
            assert torch.equal(a, t.grad)


def test_module_forward_and_causal_half():
    """HipSIRENKernelND.forward gives the reference's [1, *grid, H] (a view of the channel-first filter) and
    kernel_bhl(causal=True) the half CKConvND keeps (kernel_len // 2 onwards)."""
    torch.manual_seed(3)
    m = HipSIRENKernelND(out_dim=96, data_dim=1, mlp_hidden_dim=32, num_layers=3, embedding_dim=32, omega_0=10.0,
                         L_cache=512, use_bias=True).cuda()
    with torch.no_grad():
        for p in m.parameters():
            if p.ndim == 1:
                p.uniform_(-0.5, 0.5)  # nonzero biases
    kernel, grid = m((300,))
    assert kernel.shape == (1, 599, 96) and grid.shape == (1, 599, 1)
    pe, hl = m.positional_embedding.linear, m.hidden_linears
    ref = siren_mlp_torch(grid[0].cpu(), pe.weight.detach().cpu(), pe.bias.detach().cpu(),
                          [lin.weight.detach().cpu() for lin in hl], [lin.bias.detach().cpu() for lin in hl],
                          m.out_linear.weight.detach().cpu(), m.out_linear.bias.detach().cpu())
    assert rel_l2(ref, kernel[0]) < 1e-5
    assert kernel.movedim(-1, 1).is_contiguous()
    causal = m.kernel_bhl((300,), causal=True)
    assert causal.shape == (1, 96, 300)
    # the readout GEMM over the half may tile differently from the full one: equal to fp32 rounding
    torch.testing.assert_close(causal[0], kernel[0, 599 // 2:].t(), rtol=1e-6, atol=1e-6)


def test_unsupported_widths_raise():
    grid = torch.rand(10, 1, device="cuda")
    w0, b0, hw, hb, wo, bo = siren_params(1, 24, 32, 1, 16)
    with pytest.raises(NotImplementedError):
        siren_filter(grid, w0.cuda(), b0.cuda(), [w.cuda() for w in hw], [b.cuda() for b in hb], wo.cuda(),
                     bo.cuda())


@pytest.mark.parametrize("HD,H", [(16, 48), (32, 300), (64, 96), (128, 40)])
def test_readout_vector_paths(HD, H):
    """G a multiple of 4: the readout's 2- and 4-point-per-lane paths (HD 64 / 16, 32), and HD 128's one point per
    lane; H not a multiple of the channel block (the last block's tail rows)."""
    g = torch.Generator().manual_seed(HD)
    grid = torch.rand(4096, 2, generator=g) * 2 - 1
    w0, b0, hw, hb, wo, bo = siren_params(2, 32, HD, 2, H, bias=True, seed=HD)
    dev = lambda t: None if t is None else t.cuda()  # noqa: E731
    print(f"siren readout HD={HD} H={H}", flush=True)
    k = siren_filter(grid.cuda(), dev(w0), dev(b0), [w.cuda() for w in hw], [b.cuda() for b in hb], dev(wo),
                     dev(bo))
    ref = siren_mlp_torch(grid, w0, b0, hw, hb, wo, bo, dtype=torch.float64).t()
    assert rel_l2(ref, k) < 1e-5
    k_nb = siren_filter(grid.cuda(), dev(w0), dev(b0), [w.cuda() for w in hw], [b.cuda() for b in hb], dev(wo), None)
    ref_nb = siren_mlp_torch(grid, w0, b0, hw, hb, wo, None, dtype=torch.float64).t()
    assert rel_l2(ref_nb, k_nb) < 1e-5


# (H, HD, G, samples, bias): ragged channel counts (not a multiple of the 32-channel chunk) and point counts (not a
# multiple of 8: the element path of the loads), several samples (per-sample filters), small G (several channel
# slices, summed by the slice kernel) and a long G (one slice, many point blocks)
RB_CASES = [(256, 32, 65541, 1, True), (100, 64, 1000, 3, True), (37, 16, 729, 2, False), (4096, 32, 4096, 1, True),
            (64, 32, 33, 1, True), (300, 64, 131072, 1, False)]


@pytest.mark.parametrize("H,HD,G,nb,bias", RB_CASES)
def test_readout_backward_one_pass(H, HD, G, nb, bias):
    """nsq_siren_readout_bwd against float64 products: gact = W^T gk per sample, gW = sum_s gk_s a_s^T,
    gb = sum_s sum_g gk_s; bf16-split matrix products with fp32 accumulation stay within 2e-5 rel-L2; two calls
    are bitwise equal."""
    from nvsubquadratic_amd import _lib

    print(f"readout bwd H={H} HD={HD} G={G} nb={nb} bias={bias}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(H + G)
    gk = torch.randn(nb, H, G, device="cuda", generator=gen)
    act = torch.rand(nb, HD + 1, G, device="cuda", generator=gen) * 2 - 1
    act[:, HD] = 1.0
    wout = torch.randn(H, HD, device="cuda", generator=gen) / HD ** 0.5
    lib = _lib.get_lib()
    need = lib.nsq_siren_readout_bwd_workspace_bytes(H, HD, G, nb)
    assert need > 0

    def run():
        ws = torch.empty(need, dtype=torch.uint8, device="cuda")
        gact = torch.empty(nb, HD, G, device="cuda")
        gw = torch.empty(H, HD, device="cuda")
        gb = torch.empty(H, device="cuda") if bias else None
        _lib.check(lib.nsq_siren_readout_bwd(gk.data_ptr(), G, act.data_ptr(), G, wout.data_ptr(), H, HD, G, nb,
                                             gact.data_ptr(), gw.data_ptr(), None if gb is None else gb.data_ptr(),
                                             ws.data_ptr(), ws.numel(), _lib.stream_ptr(gk.device)))
        return gact, gw, gb

    gact, gw, gb = run()
    g64, a64, w64 = gk.double(), act[:, :HD].double(), wout.double()
    assert rel_l2(torch.matmul(w64.t(), g64), gact) < 2e-5
    assert rel_l2(torch.einsum("shg,sjg->hj", g64, a64), gw) < 2e-5
    if bias:
        assert rel_l2(g64.sum(dim=(0, 2)), gb) < 2e-5
    again = run()
    assert torch.equal(again[0], gact) and torch.equal(again[1], gw)
    if bias:
        assert torch.equal(again[2], gb)


# (d, grid shape, E, HD, nh, H, bias, samples, film_first): FiLM on the hidden layers only or also after the
# embedding (E == HD), the widths the configs use, HD = 128 (readout gradient on library products), no biases
FILM_CASES = [
    (1, (599,), 32, 32, 2, 160, True, 3, False),
    (2, (27, 27), 32, 32, 2, 384, True, 4, True),
    (3, (9, 7, 5), 16, 64, 1, 64, False, 2, False),
    (2, (13, 11), 128, 128, 3, 32, True, 2, True),
    (1, (4095,), 64, 64, 3, 256, True, 2, True),
]


@pytest.mark.parametrize("case", FILM_CASES)
def test_film_filter_matches_restatement(case):
    """FiLM-conditioned per-sample filters (kernels_nd.py:1165-1190): forward rel-L2 <= 1e-5 against float64, every
    weight, bias, gamma and beta gradient <= 1e-4 against float64 autograd, repeated backward calls bitwise equal."""
    from nvsubquadratic_amd.siren_hip import siren_film_filter
    from oracle.siren_ref import film_pairs, siren_film_torch

    d, shape, E, HD, nh, H, bias, B, ff = case
    print(f"siren film {case}", flush=True)
    grid = _grid(shape).reshape(-1, d)
    w0, b0, hw, hb, wo, bo = siren_params(d, E, HD, nh, H, bias=bias, seed=2)
    pairs = film_pairs(B, HD, nh + int(ff), seed=3)
    leaves = [w0, b0, *hw, *(hb or []), wo, bo] + [t for pr in pairs for t in pr]
    nl = len(leaves) - 2 * len(pairs)

    def split(ts):
        hb_ = ts[2 + nh:2 + 2 * nh] if hb is not None else None
        fp = [(ts[nl + 2 * i], ts[nl + 2 * i + 1]) for i in range(len(pairs))]
        return ts[0], ts[1], ts[2:2 + nh], hb_, ts[nl - 2], ts[nl - 1], fp

    ref = [None if t is None else t.double().requires_grad_(True) for t in leaves]
    w0r, b0r, hwr, hbr, wor, bor, fpr = split(ref)
    y = siren_film_torch(grid.double(), w0r, b0r, hwr, hbr, wor, bor, fpr, ff, dtype=torch.float64)  # [B, G, H]
    g = torch.randn(y.shape, dtype=torch.float64, generator=torch.Generator().manual_seed(6))
    y.backward(g)
    hip = [None if t is None else t.cuda().requires_grad_(True) for t in leaves]
    w0h, b0h, hwh, hbh, woh, boh, fph = split(hip)
    k = siren_film_filter(grid.cuda(), w0h, b0h, hwh, hbh, woh, boh, fph, ff)
    assert k.shape == (B, H, grid.shape[0])
    assert rel_l2(y.detach().transpose(1, 2), k.detach()) < 1e-5
    gk = g.transpose(1, 2).float().cuda().contiguous()
    k.backward(gk)
    first = []
    for r, h in zip(ref, hip):
        if r is None:
            continue
        assert rel_l2(r.grad, h.grad) < 1e-4
        first.append(h.grad.clone())
        h.grad = None
    siren_film_filter(grid.cuda(), w0h, b0h, hwh, hbh, woh, boh, fph, ff).backward(gk)
    assert all(torch.equal(a, h.grad) for a, h in zip(first, [t for t in hip if t is not None]))


def test_film_module_forward_and_kernel_bhl():
    """HipSIRENKernelND with film_cfg: forward(seq_lens, conditioning) -> [B, *grid, out_dim], equal to the
    restatement with the generator's own (gamma, beta); kernel_bhl gives the channel-first view; without
    conditioning the plain [1, *grid, out_dim] filter."""
    from oracle.siren_ref import siren_film_torch

    torch.manual_seed(0)
    m = HipSIRENKernelND(out_dim=48, data_dim=2, mlp_hidden_dim=32, num_layers=3, embedding_dim=32, omega_0=10.0,
                         L_cache=(14, 14), use_bias=True,
                         film_cfg=dict(cond_dim=8, kernel_hidden_dim=32, num_film_layers=3,
                                       init_type="small_random", init_std=0.2),
                         film_after_pos_embed=True).cuda()
    with torch.no_grad():
        for lin in m.hidden_linears:
            lin.bias.uniform_(-1, 1)
    cond = torch.randn(3, 8, device="cuda")
    kernel, grid = m((14, 14), conditioning=cond)
    assert kernel.shape == (3, 27, 27, 48) and grid.shape == (1, 27, 27, 2)
    pairs = [(gm.detach().cpu(), bt.detach().cpu()) for gm, bt in m.film_generator(cond)]
    pe = m.positional_embedding.linear
    ref = siren_film_torch(grid[0].reshape(-1, 2).cpu().double(), pe.weight.cpu(), pe.bias.cpu(),
                           [lin.weight.cpu() for lin in m.hidden_linears], [lin.bias.cpu() for lin in m.hidden_linears],
                           m.out_linear.weight.cpu(), m.out_linear.bias.cpu(), pairs, True, dtype=torch.float64)
    assert rel_l2(ref.reshape(3, 27, 27, 48), kernel.detach().cpu()) < 1e-5
    bhl = m.kernel_bhl((14, 14), conditioning=cond)
    assert torch.equal(bhl, kernel.movedim(-1, 1))
    plain, _ = m((14, 14))
    assert plain.shape == (1, 27, 27, 48)
    # gradients reach the FiLM generator's parameters through gamma / beta
    kernel.square().sum().backward()
    assert m.film_generator.mlp[0].weight.grad is not None and m.film_generator.mlp[0].weight.grad.abs().sum() > 0


def test_film_filters_drive_the_per_sample_causal_conv():
    """End to end: FiLM-conditioned filters [B, H, L] on the causal half of the grid feed the HIP
    causal FFT conv as per-sample filters; output and gradients (input, SIREN weights, every gamma and beta) against
    the same chain on the CPU oracle in float32, rel-L2 <= 1e-4."""
    from nvsubquadratic_amd.fftconv_hip import causal_fftconv1d_bhl
    from nvsubquadratic_amd.siren_hip import siren_film_filter
    from oracle.fftconv_ref import causal_fftconv1d_torch
    from oracle.siren_ref import film_pairs, siren_film_torch

    B, H, L, HD = 2, 64, 1024, 32
    print(f"film -> causal conv B={B} H={H} L={L}", flush=True)
    grid = siren_grid((L,), (1.0,), (L,))[L - 1:].contiguous()  # the L points CKConvND's causal crop keeps
    w0, b0, hw, hb, wo, bo = siren_params(1, 32, HD, 2, H, seed=4)
    pairs = film_pairs(B, HD, 2, seed=5)
    gen = torch.Generator().manual_seed(7)
    x = torch.randn(B, H, L, generator=gen)
    s = torch.randn(H, generator=gen)
    g = torch.randn(B, H, L, generator=gen)
    leaves = [w0, b0, *hw, *hb, wo, bo, *[t for pr in pairs for t in pr], x, s]

    def chain(ts, filt, conv, film_fn):
        w0_, b0_, w1, w2, b1, b2, wo_, bo_ = ts[:8]
        fp = [(ts[8], ts[9]), (ts[10], ts[11])]
        k = filt(film_fn, w0_, b0_, [w1, w2], [b1, b2], wo_, bo_, fp)  # [B, H, L]
        return conv(ts[12], k, ts[13])

    ref = [t.clone().requires_grad_(True) for t in leaves]
    yr = chain(ref, lambda f, *a: f(grid, *a[:6], a[6]).transpose(1, 2), causal_fftconv1d_torch, siren_film_torch)
    yr.backward(g)
    hip = [t.cuda().requires_grad_(True) for t in leaves]
    yh = chain(hip, lambda f, *a: f(grid.cuda(), *a[:6], a[6]), causal_fftconv1d_bhl, siren_film_filter)
    yh.backward(g.cuda())
    assert rel_l2(yr.detach(), yh.detach().cpu()) < 1e-4
    for r, h in zip(ref, hip):
        assert rel_l2(r.grad, h.grad.cpu()) < 1e-4
