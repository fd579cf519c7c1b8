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


if __name__ == "__main__":
    main()
