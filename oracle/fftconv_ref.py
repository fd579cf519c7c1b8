"""CPU restatement of the reference torch.fft path -- TEST INFRASTRUCTURE ONLY.

Two restatements of the same algorithm:

* ``*_torch``: float32 CPU torch, step for step the reference code
  (cast to fp32 -> ``torch.fft.rfft(n=F)`` -> complex multiply ->
  ``torch.fft.irfft(n=F)`` -> crop -> cast to ``x.dtype`` -> ``+ shortcut * x``),
  autograd-capable, so its gradients are the reference's autograd gradients.
  This is what the parity tests compare the HIP path with and what bench.py
  times as the CPU baseline.
* ``*_np``: float64 numpy version of the same steps (``numpy.fft``), used to
  separate the HIP path's error from the float32 oracle's own error.

Pinning (tests/test_oracle.py): every function here is checked against the
brute-force direct convolutions of :mod:`oracle.direct` (which use no FFT),
against the golden fixtures in ``tests/golden/``, and against closed forms
(delta and shifted-delta filters, causality, linearity, the fold at
``F = 2L`` when ``K > L + 1``).
"""

from __future__ import annotations

import numpy as np
import torch


# ---------------------------------------------------------------------------
# dtype helpers
# ---------------------------------------------------------------------------
def round_bf16_np(a: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 (round to nearest even) -> float32, in numpy."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(a), a, out)


def rel_l2(ref, test) -> float:
    """||ref - test||_2 / ||ref||_2 in float64 (nvsubquadratic/testing/utils.py:20-54)."""
    r = np.asarray(ref.detach().cpu().double() if isinstance(ref, torch.Tensor) else ref, dtype=np.float64)
    t = np.asarray(test.detach().cpu().double() if isinstance(test, torch.Tensor) else test, dtype=np.float64)
    den = np.linalg.norm(r)
    num = np.linalg.norm(r - t)
    return float(num if den < 1e-10 else num / den)


# ---------------------------------------------------------------------------
# torch (float32) restatements -- reference algorithm, CPU
# ---------------------------------------------------------------------------
def causal_fftconv1d_torch(
    x: torch.Tensor, kernel: torch.Tensor, shortcut: torch.Tensor | None = None
) -> torch.Tensor:
    """nvsubquadratic/ops/fftconv.py:546-600 (``causal_fftconv1d_fp32_bhl``) on CPU.

    Shortcut handling follows the subq wrapper, which casts the shortcut to
    ``x.dtype`` (nvsubquadratic/ops/fftconv_custom.py:333) instead of asserting
    equal dtypes (fftconv.py:597).
    """
    x_fp32 = x.to(torch.float32)
    k_fp32 = kernel.to(torch.float32)
    if k_fp32.ndim == 2:
        k_fp32 = k_fp32.unsqueeze(0)
    _B, H, L = x.shape
    K = k_fp32.shape[-1]
    assert K <= 2 * L
    F = min(L + K, 2 * L)  # fftconv.py:580
    fx = torch.fft.rfft(x_fp32, n=F, dim=2)
    fk = torch.fft.rfft(k_fp32, n=F, dim=2)
    y = torch.fft.irfft(fx * fk, n=F, dim=2)[..., :L]  # fftconv.py:591-593
    y = y.to(x.dtype)
    if shortcut is not None:
        y = y + shortcut.to(x.dtype).view(1, H, 1) * x  # fftconv_custom.py:333
    return y


def causal_fftconv1d_chunked_torch(x, kernel, shortcut=None, chunk_size=128) -> torch.Tensor:
    """Channel-chunked semantics of nvsubquadratic/ops/fftconv_chunked.py:285-322.

    Per-channel results are identical to the unchunked call; used by the CPU
    baseline to bound host memory at cfg3.
    """
    H = x.shape[1]
    if H <= chunk_size:
        return causal_fftconv1d_torch(x, kernel, shortcut)
    k = kernel if kernel.ndim == 3 else kernel.unsqueeze(0)
    outs = []
    for s in range(0, H, chunk_size):
        e = min(s + chunk_size, H)
        outs.append(
            causal_fftconv1d_torch(x[:, s:e], k[:, s:e], None if shortcut is None else shortcut[s:e])
        )
    return torch.cat(outs, dim=1)


# ---------------------------------------------------------------------------
# numpy (float64) restatements
# ---------------------------------------------------------------------------
def causal_fftconv1d_np(x, k, shortcut=None) -> np.ndarray:
    """float64 numpy version of fftconv.py:546-600 (no dtype casts, no rounding)."""
    x = np.asarray(x, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    if k.ndim == 3:
        k = k[0]
    _B, H, L = x.shape
    K = k.shape[-1]
    F = min(L + K, 2 * L)
    y = np.fft.irfft(np.fft.rfft(x, n=F, axis=-1) * np.fft.rfft(k, n=F, axis=-1)[None], n=F, axis=-1)[..., :L]
    if shortcut is not None:
        y = y + np.asarray(shortcut, dtype=np.float64)[None, :, None] * x
    return y


def causal_fftconv1d_bwd_np(g, x, k, with_shortcut: bool, shortcut=None):
    """float64 adjoint of :func:`causal_fftconv1d_np` (what autograd derives).

    gx = corr(g, k) [+ s*g], gk = sum_b corr(g_b, x_b)[:K], gs = sum g*x.
    The correlations use the same FFT length F as the forward, so the fold of
    the K > L+1 case is reproduced.
    """
    g = np.asarray(g, dtype=np.float64)
    x = np.asarray(x, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    if k.ndim == 3:
        k = k[0]
    _B, _H, L = x.shape
    K = k.shape[-1]
    F = min(L + K, 2 * L)
    G = np.fft.rfft(g, n=F, axis=-1)
    gx = np.fft.irfft(G * np.conj(np.fft.rfft(k, n=F, axis=-1))[None], n=F, axis=-1)[..., :L]
    gk = np.fft.irfft((G * np.conj(np.fft.rfft(x, n=F, axis=-1))).sum(0), n=F, axis=-1)[..., :K]
    gs = None
    if with_shortcut:
        gx = gx + np.asarray(shortcut, dtype=np.float64)[None, :, None] * g
        gs = (g * x).sum(axis=(0, 2))
    return gx, gk, gs


# ---------------------------------------------------------------------------
# 2D / 3D non-causal ("same") restatements
# ---------------------------------------------------------------------------
def fftconv_nd_torch(x: torch.Tensor, kernel: torch.Tensor, shortcut: torch.Tensor | None = None) -> torch.Tensor:
    """nvsubquadratic/ops/fftconv.py:662-733 (2D) and :736-812 (3D) on CPU float32.

    F_d = min(S_d + ceil(K_d/2), 2 S_d) per axis (:699-702 / :774-778),
    rfftn -> multiply -> irfftn -> crop [K_d//2, K_d//2 + S_d) (:714-725 /
    :789-805) -> cast to x.dtype -> + shortcut * x (shortcut cast to x.dtype as
    in the subq wrapper, fftconv_custom.py:157-158).
    """
    nd = x.ndim - 2
    if kernel.ndim == nd + 1:
        kernel = kernel.unsqueeze(0)
    H = x.shape[1]
    S = x.shape[2:]
    K = kernel.shape[2:]
    dims = tuple(range(2, 2 + nd))
    fft_shape = tuple(min(S[d] + (K[d] + 1) // 2, 2 * S[d]) for d in range(nd))
    fx = torch.fft.rfftn(x.to(torch.float32), s=fft_shape, dim=dims)
    fk = torch.fft.rfftn(kernel.to(torch.float32), s=fft_shape, dim=dims)
    y = torch.fft.irfftn(fx * fk, s=fft_shape, dim=dims)
    sl = [slice(None), slice(None)] + [slice(K[d] // 2, K[d] // 2 + S[d]) for d in range(nd)]
    y = y[tuple(sl)].to(x.dtype)
    if shortcut is not None:
        y = y + shortcut.to(x.dtype).view(1, H, *([1] * nd)) * x
    return y


def fftconv_nd_np(x, kernel, shortcut=None) -> np.ndarray:
    """float64 numpy version of :func:`fftconv_nd_torch` (power-of-two FFT sizes)."""
    x = np.asarray(x, dtype=np.float64)
    k = np.asarray(kernel, dtype=np.float64)
    nd = x.ndim - 2
    if k.ndim == nd + 1:
        k = k[None]
    S, K = x.shape[2:], k.shape[2:]
    axes = tuple(range(2, 2 + nd))
    fs = tuple(1 << int(np.ceil(np.log2(S[d] + (K[d] + 1) // 2))) for d in range(nd))
    y = np.fft.irfftn(np.fft.rfftn(x, s=fs, axes=axes) * np.fft.rfftn(k, s=fs, axes=axes), s=fs, axes=axes)
    sl = (slice(None), slice(None)) + tuple(slice(K[d] // 2, K[d] // 2 + S[d]) for d in range(nd))
    y = y[sl]
    if shortcut is not None:
        y = y + np.asarray(shortcut, dtype=np.float64).reshape((1, -1) + (1,) * nd) * x
    return y
