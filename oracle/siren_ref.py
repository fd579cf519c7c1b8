"""SIREN implicit filter (SIRENKernelND, with and without FiLM) restated on the CPU -- TEST INFRASTRUCTURE ONLY.

nvsubquadratic/modules/kernels_nd.py: the positional embedding sin(W0 x + b0) with its linear in float32
(:855-871), the hidden layers sin(W_i h + b_i) (:1181-1183; ``Sine`` is plain ``torch.sin``, :634-638),
the readout W_out h + b_out (:1189), for the coordinates ``grid [G, d]``; returns ``[G, H]`` (the
reference's ``[1, *grid, H]`` flattened).  ``dtype=torch.float64`` evaluates the same network in double
precision.  FiLM (:1165-1187): per sample b, the pair (gamma_b, beta_b) of a modulated layer maps its output h to
gamma_b * h + beta_b (broadcast over the points); with ``film_first`` the first pair modulates the positional
embedding and the rest the hidden layers in order (``film_after_pos_embed``), else one pair per hidden layer.
Pinned in tests/test_oracle_siren.py against a per-neuron loop evaluation (FiLM included), closed forms (zero hidden
weights; identity FiLM = the plain network) and float64 finite differences of its gradients.
"""

from __future__ import annotations

import torch


def siren_mlp_torch(grid, w0, b0, hidden_w, hidden_b, wout, bout, dtype=torch.float32):
    f = lambda t: None if t is None else t.to(dtype)  # noqa: E731
    h = torch.sin(torch.nn.functional.linear(grid.to(dtype), f(w0), f(b0)))
    for i, w in enumerate(hidden_w):
        h = torch.sin(torch.nn.functional.linear(h, f(w), None if hidden_b is None else f(hidden_b[i])))
    return torch.nn.functional.linear(h, f(wout), f(bout))


def siren_film_torch(grid, w0, b0, hidden_w, hidden_b, wout, bout, film_params, film_first=False,
                     dtype=torch.float32):
    """Per-sample filters ``[B, G, H]`` for the FiLM pairs ``film_params`` (each ``(gamma [B, HD], beta [B, HD])``)."""
    f = lambda t: None if t is None else t.to(dtype)  # noqa: E731
    h = torch.sin(torch.nn.functional.linear(grid.to(dtype), f(w0), f(b0)))[None]  # [1, G, E]
    pairs = [(f(g)[:, None, :], f(b)[:, None, :]) for g, b in film_params]
    off = 0
    if film_first:
        h = pairs[0][0] * h + pairs[0][1]
        off = 1
    for i, w in enumerate(hidden_w):
        h = torch.sin(torch.nn.functional.linear(h, f(w), None if hidden_b is None else f(hidden_b[i])))
        h = pairs[i + off][0] * h + pairs[i + off][1]
    return torch.nn.functional.linear(h, f(wout), f(bout))


def film_pairs(B, HD, n, seed=0):
    """Random FiLM pairs around the identity (gamma ~ 1 + U(-0.5, 0.5), beta ~ U(-0.3, 0.3)), float32."""
    g = torch.Generator().manual_seed(seed)
    return [(1 + torch.rand(B, HD, generator=g) - 0.5, (torch.rand(B, HD, generator=g) - 0.5) * 0.6)
            for _ in range(n)]


def siren_params(d, E, HD, nh, H, bias=True, omega_0=10.0, seed=0):
    """Random parameters with the reference's init scales (first layer U(+-2 pi w0 / d), hidden and readout
    U(+-sqrt(6 / fan_in))) and, for tests, nonzero biases (init sets them to zero)."""
    g = torch.Generator().manual_seed(seed)
    u = lambda shape, b: (torch.rand(*shape, generator=g) * 2 - 1) * b  # noqa: E731
    w0 = u((E, d), 2 * torch.pi * omega_0 / d)
    hw = [u((HD, E), (6 / E) ** 0.5)] + [u((HD, HD), (6 / HD) ** 0.5) for _ in range(nh - 1)]
    wout = u((H, HD), (6 / HD) ** 0.5) / 16
    if not bias:
        return w0, None, hw, None, wout, None
    b0 = u((E,), 1.0)
    hb = [u((HD,), 1.0) for _ in range(nh)]
    bout = u((H,), 0.1)
    return w0, b0, hw, hb, wout, bout
