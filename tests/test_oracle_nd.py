"""CPU pinning of the 2D / 3D FFT-conv oracle restatements (no GPU)."""

import os

import numpy as np
import pytest
import torch

from oracle import direct
from oracle.fftconv_ref import fftconv_nd_np, fftconv_nd_torch, rel_l2


GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "nd.npz")
CASES = [((2, 3, 9, 7), (5, 3)), ((1, 2, 16, 16), (16, 16)), ((1, 2, 6, 5), (12, 9)), ((1, 2, 14, 14), (28, 28)),
         ((1, 2, 5, 6, 7), (3, 4, 5)), ((1, 1, 4, 4, 4), (8, 1, 7)), ((1, 1, 6, 6, 6), (2, 2, 2))]


@pytest.mark.parametrize("xs,ks", CASES)
def test_restatements_match_brute_force(xs, ks):
    rng = np.random.default_rng(len(xs) * 10 + ks[0])
    x = rng.standard_normal(xs)
    k = rng.standard_normal((xs[1],) + ks)
    s = rng.standard_normal(xs[1])
    ref = direct.conv_same_nd(x, k) + s.reshape((1, -1) + (1,) * len(ks)) * x
    assert rel_l2(ref, fftconv_nd_np(x, k, s)) < 1e-12
    yt = fftconv_nd_torch(torch.tensor(x, dtype=torch.float32), torch.tensor(k, dtype=torch.float32),
                          torch.tensor(s, dtype=torch.float32))
    assert rel_l2(ref, yt) < 1e-5


def test_golden_fixtures():
    d = np.load(GOLDEN)
    for i in range(int(d["n_nd"])):
        x, k, s = d[f"n{i}_x"], d[f"n{i}_k"], d[f"n{i}_s"]
        nd = x.ndim - 2
        assert rel_l2(direct.conv_same_nd(x, k) + s.reshape((1, -1) + (1,) * nd) * x, d[f"n{i}_y"]) < 1e-13
        assert rel_l2(d[f"n{i}_y"], fftconv_nd_np(x, k, s)) < 1e-12


def test_centered_delta_is_identity():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((1, 2, 10, 9))
    k = np.zeros((2, 7, 5))
    k[:, 3, 2] = 1.0  # index K//2 is the zero-lag tap after the crop
    np.testing.assert_allclose(fftconv_nd_np(x, k), x, atol=1e-12)


def test_rank_one_kernel_is_separable():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((1, 1, 12, 11))
    a, b = rng.standard_normal(5), rng.standard_normal(4)
    k = np.outer(a, b)[None]
    # successive 1D 'same' convolutions along each axis (brute force)
    t = direct.conv_same_nd(np.transpose(x, (0, 1, 3, 2)).reshape(1, 11, 12), np.tile(a, (11, 1)))
    t = np.transpose(t.reshape(1, 1, 11, 12), (0, 1, 3, 2))
    t = direct.conv_same_nd(t.reshape(1, 12, 11), np.tile(b, (12, 1))).reshape(1, 1, 12, 11)
    assert rel_l2(t, fftconv_nd_np(x, k)) < 1e-12
