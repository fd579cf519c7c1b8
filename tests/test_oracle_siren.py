"""Pins the SIREN restatement (oracle/siren_ref.py) -- CPU only."""

import math

import pytest
import torch

from nvsubquadratic_amd.siren_hip import HipSIRENKernelND, siren_grid
from oracle.siren_ref import film_pairs, siren_film_torch, siren_mlp_torch, siren_params


def _loops(grid, w0, b0, hw, hb, wout, bout):
    """Per-neuron evaluation with Python loops in float64 (no matrix products)."""
    G, d = grid.shape
    out = torch.zeros(G, wout.shape[0], dtype=torch.float64)
    for g in range(G):
        x = [float(v) for v in grid[g]]
        h = [math.sin(sum(float(w0[e, c]) * x[c] for c in range(d)) + (float(b0[e]) if b0 is not None else 0.0))
             for e in range(w0.shape[0])]
        for i, w in enumerate(hw):
            h = [math.sin(sum(float(w[o, j]) * h[j] for j in range(len(h))) + (float(hb[i][o]) if hb else 0.0))
                 for o in range(w.shape[0])]
        for c in range(wout.shape[0]):
            out[g, c] = sum(float(wout[c, j]) * h[j] for j in range(len(h))) + (float(bout[c]) if bout is not None
                                                                               else 0.0)
    return out


@pytest.mark.parametrize("d,nh,bias", [(1, 1, True), (2, 2, True), (3, 3, False)])
def test_restatement_matches_per_neuron_loops(d, nh, bias):
    params = siren_params(d, 4, 5, nh, 3, bias=bias, seed=d)
    grid = torch.rand(6, d, dtype=torch.float64) * 2 - 1
    ref = _loops(grid, *params)
    assert torch.allclose(siren_mlp_torch(grid, *params, dtype=torch.float64), ref, rtol=1e-12, atol=1e-12)


def test_zero_hidden_weights_give_a_constant_filter():
    w0, b0, hw, hb, wout, bout = siren_params(1, 8, 8, 2, 4, seed=3)
    hw = [torch.zeros_like(w) for w in hw]
    grid = torch.linspace(-1, 1, 11).unsqueeze(1)
    k = siren_mlp_torch(grid, w0, b0, hw, hb, wout, bout, dtype=torch.float64)
    closed = wout.double() @ torch.sin(hb[-1].double()) + bout.double()
    assert torch.allclose(k, closed.expand_as(k), rtol=1e-12, atol=1e-12)


def test_restatement_gradients_match_finite_differences():
    params = [p.double().requires_grad_(True) if p is not None else None for p in
              (lambda w0, b0, hw, hb, wo, bo: [w0, b0, *hw, *hb, wo, bo])(*siren_params(2, 4, 4, 2, 3, seed=4))]
    grid = torch.rand(5, 2, dtype=torch.float64) * 2 - 1

    def f(w0, b0, w1, w2, b1, b2, wo, bo):
        return siren_mlp_torch(grid, w0, b0, [w1, w2], [b1, b2], wo, bo, dtype=torch.float64)

    assert torch.autograd.gradcheck(f, tuple(params), eps=1e-6, atol=1e-7)


def test_grid_is_the_caches_central_points_at_the_original_step():
    """Cache linspace(-1, 1, 2L - 1): the central 2s - 1 points are (k - (s - 1)) / (L - 1); past the cache the
    axis grows with the original step (kernels_nd.py:780-815)."""
    L, s = 16, 5
    g = siren_grid((L,), (1.0,), (s,))[:, 0].double()
    closed = (torch.arange(2 * s - 1, dtype=torch.float64) - (s - 1)) / (L - 1)
    assert torch.allclose(g, closed, atol=1e-7)
    m = HipSIRENKernelND(16, 1, 16, 2, 16, 10.0, L, True)
    g2 = m._grid((20,))[:, 0].double()
    closed2 = (torch.arange(39, dtype=torch.float64) - 19) / (L - 1)
    assert torch.allclose(g2, closed2, atol=1e-6)
    assert m.L_cache_per_axis == (20,)


def test_module_init_and_parameter_names_follow_the_reference():
    """Parameter names of SIRENKernelND (state dicts interchange) and its init bounds: first layer
    |W| <= 2 pi w0 / d, hidden |W| <= sqrt(6 / fan_in), readout additionally scaled by sqrt(1 / prod(L_cache))."""
    torch.manual_seed(0)
    m = HipSIRENKernelND(out_dim=32, data_dim=2, mlp_hidden_dim=32, num_layers=3, embedding_dim=16, omega_0=10.0,
                         L_cache=(8, 4), use_bias=True)
    names = sorted(m.state_dict())
    assert names == ["hidden_linears.0.bias", "hidden_linears.0.weight", "hidden_linears.1.bias",
                     "hidden_linears.1.weight", "out_linear.bias", "out_linear.weight",
                     "positional_embedding.linear.bias", "positional_embedding.linear.weight"]
    assert m.positional_embedding.linear.weight.abs().max() <= 2 * math.pi * 10.0 / 2
    assert m.hidden_linears[0].weight.abs().max() <= math.sqrt(6 / 16)
    assert m.out_linear.weight.abs().max() <= math.sqrt(6 / 32) * math.sqrt(1 / 32)
    assert all(float(b.abs().max()) == 0.0 for b in (m.out_linear.bias, m.hidden_linears[0].bias))
    with pytest.raises(TypeError):
        HipSIRENKernelND(32, 1, 32, 3, 32, 10.0, 8, True, film_cfg=object())


def _film_loops(grid, w0, b0, hw, hb, wout, bout, pairs, film_first):
    """Per-neuron float64 loops with FiLM: sample b's pair maps each modulated neuron's output v to g_b v + beta_b."""
    B = pairs[0][0].shape[0]
    out = torch.zeros(B, grid.shape[0], wout.shape[0], dtype=torch.float64)
    for b in range(B):
        for g in range(grid.shape[0]):
            x = [float(v) for v in grid[g]]
            h = [math.sin(sum(float(w0[e, c]) * x[c] for c in range(len(x))) + (float(b0[e]) if b0 is not None
                                                                                else 0.0)) for e in range(w0.shape[0])]
            k = 0
            if film_first:
                h = [float(pairs[0][0][b, e]) * h[e] + float(pairs[0][1][b, e]) for e in range(len(h))]
                k = 1
            for i, w in enumerate(hw):
                h = [math.sin(sum(float(w[o, j]) * h[j] for j in range(len(h))) + (float(hb[i][o]) if hb else 0.0))
                     for o in range(w.shape[0])]
                gm, bt = pairs[i + k]
                h = [float(gm[b, o]) * h[o] + float(bt[b, o]) for o in range(len(h))]
            for c in range(wout.shape[0]):
                out[b, g, c] = sum(float(wout[c, j]) * h[j] for j in range(len(h))) + (float(bout[c]) if bout is not
                                                                                       None else 0.0)
    return out


@pytest.mark.parametrize("film_first", [False, True])
def test_film_restatement_matches_per_neuron_loops(film_first):
    params = siren_params(2, 5, 5, 2, 3, seed=7)
    pairs = film_pairs(2, 5, 2 + int(film_first), seed=8)
    grid = torch.rand(4, 2, dtype=torch.float64) * 2 - 1
    ref = _film_loops(grid, *params, pairs, film_first)
    got = siren_film_torch(grid, *params, pairs, film_first, dtype=torch.float64)
    assert torch.allclose(got, ref, rtol=1e-12, atol=1e-12)


def test_identity_film_is_the_plain_network_and_zero_weights_give_constants():
    w0, b0, hw, hb, wout, bout = siren_params(1, 8, 8, 2, 4, seed=9)
    grid = torch.linspace(-1, 1, 9).unsqueeze(1).double()
    ident = [(torch.ones(3, 8), torch.zeros(3, 8)) for _ in range(3)]
    plain = siren_mlp_torch(grid, w0, b0, hw, hb, wout, bout, dtype=torch.float64)
    film = siren_film_torch(grid, w0, b0, hw, hb, wout, bout, ident, True, dtype=torch.float64)
    assert torch.equal(film, plain.expand_as(film))
    # zero hidden weights: h_nh = gamma_nh sin(b_nh) + beta_nh per sample, a constant filter per sample
    pairs = film_pairs(3, 8, 2, seed=10)
    zero = [torch.zeros_like(w) for w in hw]
    k = siren_film_torch(grid, w0, b0, zero, hb, wout, bout, pairs, False, dtype=torch.float64)
    h = pairs[1][0].double() * torch.sin(hb[-1].double()) + pairs[1][1].double()  # [3, 8]
    closed = h @ wout.double().t() + bout.double()
    assert torch.allclose(k, closed[:, None, :].expand_as(k), rtol=1e-12, atol=1e-12)


def test_film_restatement_gradients_match_finite_differences():
    w0, b0, hw, hb, wout, bout = [p for p in siren_params(1, 4, 4, 2, 3, seed=11)]
    pairs = film_pairs(2, 4, 3, seed=12)
    grid = torch.rand(5, 1, dtype=torch.float64) * 2 - 1
    leaves = [t.double().requires_grad_(True) for t in (w0, b0, *hw, *hb, wout, bout)] + \
             [t.double().requires_grad_(True) for pr in pairs for t in pr]

    def f(*ts):
        w0_, b0_, w1, w2, b1, b2, wo, bo = ts[:8]
        fp = [(ts[8 + 2 * i], ts[9 + 2 * i]) for i in range(3)]
        return siren_film_torch(grid, w0_, b0_, [w1, w2], [b1, b2], wo, bo, fp, True, dtype=torch.float64)

    assert torch.autograd.gradcheck(f, tuple(leaves), eps=1e-6, atol=1e-7)


def test_film_generator_follows_the_reference():
    """KernelFiLMGenerator (modules/film.py:75): parameter names, identity init (gamma = 1, beta = 0), output split
    per layer, weight-decay flags; HipSIRENKernelND checks the layer count and film_after_pos_embed's width rule."""
    from nvsubquadratic_amd.siren_hip import KernelFiLMGenerator

    torch.manual_seed(0)
    g = KernelFiLMGenerator(cond_dim=6, kernel_hidden_dim=4, num_film_layers=3, film_hidden_dim=5)
    assert sorted(n for n, _ in g.named_parameters()) == ["mlp.0.bias", "mlp.0.weight", "mlp.2.bias", "mlp.2.weight"]
    pairs = g(torch.randn(2, 6))
    assert len(pairs) == 3 and all(gm.shape == (2, 4) and bt.shape == (2, 4) for gm, bt in pairs)
    assert all(torch.equal(gm, torch.ones(2, 4)) and torch.equal(bt, torch.zeros(2, 4)) for gm, bt in pairs)
    assert g.mlp[0].bias._no_weight_decay and g.mlp[2].bias._no_weight_decay
    assert not getattr(g.mlp[0].weight, "_no_weight_decay", False)
    assert KernelFiLMGenerator(6, 4, 1, no_weight_decay=1e-3).mlp[0].weight._weight_decay == 1e-3
    r = KernelFiLMGenerator(6, 4, 2, init_type="small_random", init_std=1e-2)
    assert 0 < float(r.mlp[2].weight.abs().max()) < 0.1
    with pytest.raises(ValueError):
        KernelFiLMGenerator(6, 4, 0)
    with pytest.raises(ValueError):
        KernelFiLMGenerator(6, 4, 1, init_type="other")
    with pytest.raises(ValueError, match="does not match expected 3"):
        HipSIRENKernelND(16, 1, 8, 3, 8, 10.0, 8, True, film_cfg=dict(cond_dim=4, kernel_hidden_dim=8,
                                                                        num_film_layers=2), film_after_pos_embed=True)
    with pytest.raises(AssertionError, match="film_after_pos_embed requires"):
        HipSIRENKernelND(16, 1, 8, 3, 16, 10.0, 8, True, film_after_pos_embed=True)
    m = HipSIRENKernelND(16, 1, 8, 3, 8, 10.0, 8, True, film_cfg=dict(cond_dim=4, kernel_hidden_dim=8,
                                                                        num_film_layers=3), film_after_pos_embed=True)
    assert "film_generator.mlp.2.weight" in m.state_dict()
