"""Writes the golden fixtures in this directory from the brute-force oracle.

The reference repository ships no stored vectors for this path (all of its
tests draw seeded random inputs and compare against closed-form spatial
convolutions, tests/ops/test_fftconv.py:68-101).  These fixtures are the same
closed forms evaluated once in float64 by oracle/direct_conv.c (no FFT
involved) on small seeded inputs, so the FFT restatement and the HIP kernels
are both checked against values computed without any FFT.

Run:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
import sys

import numpy as np


HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import direct  # noqa: E402


# (B, H, L, K): reference test shapes scaled down, K == L, odd L, K > L+1 (fold)
CAUSAL_CASES = [
    (2, 4, 64, 7),
    (1, 3, 32, 32),
    (2, 2, 16, 3),
    (1, 2, 17, 5),
    (1, 2, 16, 24),  # K > L+1: the reference FFT length 2L wraps
    (1, 2, 9, 18),  # K == 2L, maximal wrap
    (3, 1, 40, 1),  # single tap
]


def _f32(a):
    return a.astype(np.float32).astype(np.float64)


# (B, C, L, K) for the direct depthwise causal conv; K up to the 256-tap limit
DIRECT_CASES = [(2, 16, 64, 3), (2, 36, 256, 3), (2, 64, 128, 7), (1, 3, 40, 64), (1, 2, 300, 256), (3, 2, 5, 9)]
# (B, C, L, Kp, Km) for the B2B block
B2B_CASES = [(2, 4, 64, 3, 3), (1, 3, 100, 4, 16), (2, 2, 70, 8, 128)]


# (B, H, S..., K...) for the 2D / 3D non-causal "same" conv
ND_CASES = [((2, 3, 9, 7), (5, 3)), ((1, 2, 16, 16), (16, 16)), ((1, 2, 6, 5), (12, 9)),
            ((1, 2, 5, 6, 7), (3, 4, 5)), ((2, 1, 4, 4, 4), (8, 1, 7))]


def nd_fixtures(rng) -> dict:
    out = {}
    for i, (xs, ks) in enumerate(ND_CASES):
        x = _f32(rng.standard_normal(xs))
        k = _f32(rng.standard_normal((xs[1],) + ks))
        s = _f32(rng.standard_normal(xs[1]))
        y = direct.conv_same_nd(x, k) + s.reshape((1, -1) + (1,) * len(ks)) * x
        for name, v in dict(x=x, k=k, s=s, y=y).items():
            out[f"n{i}_{name}"] = v
    out["n_nd"] = np.array(len(ND_CASES))
    return out


def _silu(v):
    return v / (1.0 + np.exp(-v))


def direct_fixtures(rng) -> dict:
    out = {}
    for i, (B, C, L, K) in enumerate(DIRECT_CASES):
        x = _f32(rng.standard_normal((B, C, L)))
        w = _f32(rng.standard_normal((C, K)) / np.sqrt(K))
        b = _f32(rng.standard_normal(C))
        pre = direct.direct_causal_conv1d(x, w, b)
        for name, v in dict(x=x, w=w, b=b, y=pre, y_silu=_silu(pre)).items():
            out[f"d{i}_{name}"] = v
        out[f"d{i}_shape"] = np.array([B, C, L, K])
    out["n_direct"] = np.array(len(DIRECT_CASES))
    for i, (B, C, L, Kp, Km) in enumerate(B2B_CASES):
        x = _f32(rng.standard_normal((B, 3 * C, L)))
        wp = _f32(rng.standard_normal((3 * C, Kp)) / np.sqrt(Kp))
        wm = _f32(rng.standard_normal((C, Km)) / np.sqrt(Km))
        sk = _f32(rng.standard_normal(C))
        p = direct.direct_causal_conv1d(x, wp)
        q, k, v = p[:, :C], p[:, C:2 * C], p[:, 2 * C:]
        z = k * v
        y = q * (direct.direct_causal_conv1d(z, wm) + sk[None, :, None] * z)
        for name, val in dict(x=x, wp=wp, wm=wm, skip=sk, y=y).items():
            out[f"b{i}_{name}"] = val
        out[f"b{i}_shape"] = np.array([B, C, L, Kp, Km])
    out["n_b2b"] = np.array(len(B2B_CASES))
    return out


def main() -> None:
    rng = np.random.default_rng(1234)
    out = {}
    for i, (B, H, L, K) in enumerate(CAUSAL_CASES):
        x = _f32(rng.standard_normal((B, H, L)))
        k = _f32(rng.standard_normal((H, K)))
        s = _f32(rng.standard_normal(H))
        g = _f32(rng.standard_normal((B, H, L)))
        y = direct.causal_conv1d(x, k) + s[None, :, None] * x
        gx, gk = direct.causal_conv1d_bwd(g, x, k)
        gx = gx + s[None, :, None] * g
        gs = (g * x).sum(axis=(0, 2))
        for name, v in dict(x=x, k=k, s=s, g=g, y=y, gx=gx, gk=gk, gs=gs).items():
            out[f"c{i}_{name}"] = v
        out[f"c{i}_shape"] = np.array([B, H, L, K])
    out["n_causal"] = np.array(len(CAUSAL_CASES))
    np.savez_compressed(os.path.join(HERE, "causal1d.npz"), **out)
    print("wrote", os.path.join(HERE, "causal1d.npz"), len(CAUSAL_CASES), "cases")
    d = direct_fixtures(np.random.default_rng(4321))
    np.savez_compressed(os.path.join(HERE, "direct1d.npz"), **d)
    print("wrote", os.path.join(HERE, "direct1d.npz"), len(DIRECT_CASES), "direct +", len(B2B_CASES), "b2b cases")
    n = nd_fixtures(np.random.default_rng(99))
    np.savez_compressed(os.path.join(HERE, "nd.npz"), **n)
    print("wrote", os.path.join(HERE, "nd.npz"), len(ND_CASES), "2D/3D cases")


if __name__ == "__main__":
    main()
