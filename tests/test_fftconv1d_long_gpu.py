"""GPU parity of the 1D convs at FFT length 2^24, the longest the 4-step plan takes (N = 2048 x 4096: 2048-point
column passes of 8 columns per 1024-thread workgroup, 4096-point row pairs).

Causal: L = 2^22 + 4096 with K = L (L + K - 1 > 2^23), so the reference's FFT length min(L + K, 2L) = 2L runs at
2^24 here; shared filters at B = 1 (the single-tile row adjoint) and B = 2 (the two-tile one, the filter gradient
summed over the batch), and per-sample filters; fp32 and bf16 I/O.  Non-causal "same": L + ceil(K/2) just below
2^24.  The oracle is float64 numpy on the same (rounded) inputs: the reference's own FFT length and formula
(``oracle/fftconv_ref.py``: ``nvsubquadratic/ops/fftconv.py:546-600``), and for "same" the full linear convolution
sliced at [K//2, K//2 + L) (``fftconv.py:603-660``).  Tolerances: 1e-4 rel-L2 for fp32 results, 5e-3 for values
rounded to bf16 (its rounding alone is ~2e-3).
"""

import numpy as np
import pytest
import torch
from scipy.signal import fftconvolve

from nvsubquadratic_amd import fftconv_hip as F
from oracle.fftconv_ref import causal_fftconv1d_bwd_np, causal_fftconv1d_np, rel_l2

pytestmark = pytest.mark.gpu

L24 = (1 << 22) + 4096


@pytest.mark.parametrize("B,H,kb,dtype", [(1, 2, 1, torch.float32), (2, 1, 1, torch.bfloat16),
                                          (2, 1, 2, torch.float32)])
def test_causal_fft_length_2_24(B, H, kb, dtype):
    L = K = L24
    print(f"causal 1D at FFT 2^24 B={B} H={H} kb={kb} {dtype}", flush=True)
    gen = torch.Generator().manual_seed(B * 10 + kb)
    t = torch.arange(K, dtype=torch.float32)
    x = torch.randn(B, H, L, generator=gen).to(dtype)
    k = torch.randn(kb, H, K, generator=gen) * torch.exp(-4.0 * t / K)
    s = torch.randn(H, generator=gen).to(dtype)
    g = torch.randn(B, H, L, generator=gen).to(dtype)
    xg, kg, sg = (v.cuda().requires_grad_(True) for v in (x, k, s))
    y = F.causal_fftconv1d_bhl(xg, kg, sg)
    y.backward(g.cuda())
    x64, k64, s64, g64 = (v.double().numpy() for v in (x, k, s, g))
    if kb == 1:
        y64 = causal_fftconv1d_np(x64, k64, s64)
        gx64, gk64, gs64 = causal_fftconv1d_bwd_np(g64, x64, k64, True, s64)
        gk64 = gk64[None]
    else:  # per-sample filters: each image with its own filter, the shortcut gradient summed over the images
        parts = [causal_fftconv1d_bwd_np(g64[b:b + 1], x64[b:b + 1], k64[b], True, s64) for b in range(B)]
        y64 = np.concatenate([causal_fftconv1d_np(x64[b:b + 1], k64[b], s64) for b in range(B)])
        gx64 = np.concatenate([p[0] for p in parts])
        gk64 = np.stack([p[1] for p in parts])
        gs64 = sum(p[2] for p in parts)
    tol = 1e-4 if dtype == torch.float32 else 5e-3
    assert rel_l2(y64, y) < tol
    assert rel_l2(gx64, xg.grad) < tol
    assert rel_l2(gk64, kg.grad) < 1e-4  # filter gradient in fp32 whatever the I/O dtype
    assert rel_l2(gs64, sg.grad) < tol


def test_same_fft_length_2_24():
    B, H, L, K = 1, 2, (1 << 24) - 600, 1000  # L + ceil(K/2) = 2^24 - 100
    print(f"same 1D at FFT 2^24 L={L} K={K}", flush=True)
    rng = np.random.default_rng(24)
    x = rng.standard_normal((B, H, L)).astype(np.float32)
    k = (rng.standard_normal((1, H, K)) / K ** 0.5).astype(np.float32)
    s = rng.standard_normal(H).astype(np.float32)
    y = F.fftconv1d_bhl(torch.tensor(x).cuda(), torch.tensor(k).cuda(), torch.tensor(s).cuda())
    c = K // 2
    ref = np.stack([fftconvolve(x[0, h].astype(np.float64), k[0, h].astype(np.float64))[c:c + L] for h in range(H)])
    ref = ref[None] + s.astype(np.float64)[None, :, None] * x
    assert rel_l2(ref, y) < 1e-4
