"""CPU pinning of the direct-conv and B2B oracle restatements (no GPU)."""

import os

import numpy as np
import pytest
import torch

from oracle import direct
from oracle.direct_ref import b2b_causal_conv1d_torch, causal_conv1d_torch
from oracle.fftconv_ref import rel_l2


GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "direct1d.npz")


@pytest.mark.parametrize("B,C,L,K", [(2, 16, 64, 3), (1, 4, 33, 256), (2, 3, 7, 9)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_causal_conv1d_torch_matches_brute_force(B, C, L, K, with_bias):
    rng = np.random.default_rng(B * 100 + K)
    x = rng.standard_normal((B, C, L))
    w = rng.standard_normal((C, K))
    b = rng.standard_normal(C) if with_bias else None
    y = causal_conv1d_torch(torch.tensor(x), torch.tensor(w), None if b is None else torch.tensor(b))
    assert rel_l2(direct.direct_causal_conv1d(x, w, b), y) < 1e-12


def test_silu_and_fixtures():
    d = np.load(GOLDEN)
    for i in range(int(d["n_direct"])):
        x, w, b = (torch.tensor(d[f"d{i}_{n}"]) for n in ("x", "w", "b"))
        assert rel_l2(direct.direct_causal_conv1d(d[f"d{i}_x"], d[f"d{i}_w"], d[f"d{i}_b"]), d[f"d{i}_y"]) < 1e-13
        assert rel_l2(d[f"d{i}_y"], causal_conv1d_torch(x, w, b)) < 1e-12
        assert rel_l2(d[f"d{i}_y_silu"], causal_conv1d_torch(x, w, b, "silu")) < 1e-12


def test_b2b_torch_matches_fixtures():
    d = np.load(GOLDEN)
    for i in range(int(d["n_b2b"])):
        x, wp, wm, sk = (torch.tensor(d[f"b{i}_{n}"]) for n in ("x", "wp", "wm", "skip"))
        y = b2b_causal_conv1d_torch(x, wp, wm, sk)
        assert rel_l2(d[f"b{i}_y"], y) < 1e-6  # the restatement computes in fp32


def test_b2b_delta_weights_closed_form():
    # identity taps (w[..., K-1] = 1): p = x, h = z + skip*z -> y = q*k*v*(1+skip)
    rng = np.random.default_rng(5)
    B, C, L = 2, 3, 20
    x = torch.tensor(rng.standard_normal((B, 3 * C, L)))
    wp = torch.zeros(3 * C, 4, dtype=torch.float64)
    wp[:, -1] = 1
    wm = torch.zeros(C, 5, dtype=torch.float64)
    wm[:, -1] = 1
    sk = torch.tensor(rng.standard_normal(C))
    y = b2b_causal_conv1d_torch(x, wp, wm, sk)
    q, k, v = x[:, :C], x[:, C:2 * C], x[:, 2 * C:]
    expect = q * k * v * (1 + sk.view(1, C, 1))
    assert rel_l2(expect, y) < 1e-6
