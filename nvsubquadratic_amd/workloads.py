"""Seeded synthetic inputs for the benchmark configurations of the hot path.

Distributions follow the benchmark configuration strings (five configs: 1D
causal fp32, B2B bf16, 1D causal long-context, 2D and 3D non-causal); all
tensors come from a ``torch.Generator`` seeded with ``seed`` on ``device``, so
a CPU checker and the GPU path see identical values when both are generated
on the CPU and moved.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch


__all__ = [
    "Causal1DCase",
    "algorithmic_bytes_b2b",
    "algorithmic_bytes_causal1d",
    "algorithmic_bytes_nd",
    "causal1d_case",
    "causal1d_case_fast",
    "decaying_filter_1d",
    "fft_flops_causal1d",
    "radial_filter",
]


@dataclass
class Causal1DCase:
    x: torch.Tensor  # [B, H, L]
    k: torch.Tensor  # [H, L] float32
    s: torch.Tensor  # [H] in x.dtype
    g: torch.Tensor  # [B, H, L] upstream gradient in x.dtype


def decaying_filter_1d(H: int, L: int, a_lo: float, a_hi: float, gen: torch.Generator, device) -> torch.Tensor:
    """h[d, t] = N(0,1) * exp(-a_d * t / L), a_d ~ U(a_lo, a_hi); float32 [H, L]."""
    a = torch.empty(H, 1, device=device).uniform_(a_lo, a_hi, generator=gen)
    t = torch.arange(L, device=device, dtype=torch.float32).view(1, L)
    h = torch.randn(H, L, device=device, generator=gen)
    return h * torch.exp(-a * t / L)


def causal1d_case(
    B: int,
    H: int,
    L: int,
    dtype: torch.dtype,
    a_range: tuple[float, float],
    device="cpu",
    seed: int = 0,
    channels: slice | None = None,
) -> Causal1DCase:
    """1D causal FFT long-conv inputs (configs 1 and 3 of the benchmark set).

    ``channels`` selects a channel subset *after* generating the full-size
    filter statistics per channel; it is used to give the CPU checker a
    bounded sample of the same workload.  Values for a channel do not depend
    on whether a subset is taken (each channel is drawn from its own stream).
    """
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    hs = range(H) if channels is None else range(*channels.indices(H))
    xs, ks, ss, gs = [], [], [], []
    # Per-channel streams: seed + 1 + h keeps a channel's values independent of H.
    for h in hs:
        gh = torch.Generator(device=device)
        gh.manual_seed(seed * 1_000_003 + 1 + h)
        xs.append(torch.randn(B, 1, L, device=device, generator=gh))
        a = torch.empty(1, 1, device=device).uniform_(a_range[0], a_range[1], generator=gh)
        t = torch.arange(L, device=device, dtype=torch.float32).view(1, L)
        ks.append(torch.randn(1, L, device=device, generator=gh) * torch.exp(-a * t / L))
        ss.append(torch.randn(1, device=device, generator=gh))
        gs.append(torch.randn(B, 1, L, device=device, generator=gh))
    x = torch.cat(xs, dim=1).to(dtype)
    k = torch.cat(ks, dim=0)
    s = torch.cat(ss).to(dtype)
    g = torch.cat(gs, dim=1).to(dtype)
    del gen
    return Causal1DCase(x=x, k=k, s=s, g=g)


def causal1d_case_fast(B: int, H: int, L: int, dtype: torch.dtype, a_range, device, seed: int = 0) -> Causal1DCase:
    """Same distributions as :func:`causal1d_case`, generated in bulk on ``device``.

    Used for the full-size benchmark (config 3: 2^30 elements per tensor) where
    per-channel generation would be slow; values differ from the per-channel
    generator but follow the same distributions.
    """
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    x = torch.randn(B, H, L, device=device, generator=gen).to(dtype)
    a = torch.empty(H, 1, device=device).uniform_(a_range[0], a_range[1], generator=gen)
    k = torch.randn(H, L, device=device, generator=gen)
    k.mul_(torch.exp(-a * torch.arange(L, device=device, dtype=torch.float32).view(1, L) / L))
    s = torch.randn(H, device=device, generator=gen).to(dtype)
    g = torch.randn(B, H, L, device=device, generator=gen).to(dtype)
    return Causal1DCase(x=x, k=k, s=s, g=g)


def algorithmic_bytes_causal1d(B: int, H: int, L: int, K: int, itemsize: int, phase: str) -> int:
    """Compulsory HBM bytes of one causal FFT-conv call (each input read once,
    each output written once; spectra and intermediates excluded).

    fwd: x read + y written (itemsize per element), k read (4 B per tap),
         shortcut read (itemsize per channel).
    bwd: g, x read + gx written (itemsize per element), k read + gk written
         (4 B per tap each), shortcut read + its gradient written (itemsize
         per channel each).
    For config 3 (B=1, H=4096, L=K=262144, bf16) this is 8,589,942,784 B
    forward and 15,032,401,920 B backward.
    """
    E = B * H * L
    if phase == "fwd":
        return E * 2 * itemsize + H * K * 4 + H * itemsize
    if phase == "bwd":
        return E * 3 * itemsize + H * K * 8 + 2 * H * itemsize
    if phase == "fwd+bwd":
        return algorithmic_bytes_causal1d(B, H, L, K, itemsize, "fwd") + algorithmic_bytes_causal1d(
            B, H, L, K, itemsize, "bwd"
        )
    raise ValueError(phase)


def fft_flops_causal1d(B: int, H: int, L: int, K: int, phase: str) -> float:
    """Radix-2 real-FFT operation count, 2.5 * F * log2(F) per length-F real
    transform (reported next to GB/s; not the metric).

    fwd: B*H forward (x) + H forward (k) + B*H inverse.
    bwd: B*H (g) + B*H (x) + H (k) forward, B*H (gx) + H (gk) inverse.
    """
    F = 1 << max(4, math.ceil(math.log2(max(L + K - 1, 2))))
    per = 2.5 * F * math.log2(F)
    if phase == "fwd":
        return (2 * B * H + H) * per
    if phase == "bwd":
        return (3 * B * H + 2 * H) * per
    if phase == "fwd+bwd":
        return (5 * B * H + 3 * H) * per
    raise ValueError(phase)


def radial_filter(C: int, size: int, sig_lo: float, sig_hi: float, nd: int, gen: torch.Generator,
                  device="cpu") -> torch.Tensor:
    """Per-channel ND filter N(0,1) * exp(-r / sigma_c), r = distance from the
    centre (size // 2 along each axis), sigma_c ~ U(sig_lo, sig_hi); float32
    [C, size, ..., size] (configs 4 and 5)."""
    sig = torch.empty(C, device=device).uniform_(sig_lo, sig_hi, generator=gen)
    ax = torch.arange(size, device=device).float() - size // 2
    grids = torch.meshgrid(*([ax] * nd), indexing="ij")
    r = torch.sqrt(sum(g ** 2 for g in grids))
    h = torch.randn(C, *([size] * nd), device=device, generator=gen)
    return h * torch.exp(-r[None] / sig.view(-1, *([1] * nd)))


def algorithmic_bytes_b2b(B: int, C: int, L: int, Kp: int, Km: int, itemsize: int, phase: str = "fwd") -> int:
    """Compulsory HBM bytes of the fused B2B block.

    Forward: x [B, 3C, L] read, y [B, C, L] written (itemsize each), fp32
    depthwise weights [3C, Kp] and [C, Km] read.  Config 2 (B=4, C=4096,
    L=8192, Kp=3, Km=128, bf16): 1,075,986,432 B.  Backward: g [B, C, L] and x
    read, gx [B, 3C, L] written, the weights and the skip [C] read and their
    fp32 gradients written."""
    E = B * C * L
    W = 3 * C * Kp + C * Km
    if phase == "fwd":
        return 3 * E * itemsize + E * itemsize + W * 4
    if phase == "bwd":
        return E * itemsize + 3 * E * itemsize + 3 * E * itemsize + 2 * (W + C) * 4
    if phase == "fwd+bwd":
        return algorithmic_bytes_b2b(B, C, L, Kp, Km, itemsize, "fwd") + algorithmic_bytes_b2b(
            B, C, L, Kp, Km, itemsize, "bwd")
    raise ValueError(phase)


def algorithmic_bytes_nd(B: int, C: int, S, K, itemsize: int, phase: str) -> int:
    """Compulsory HBM bytes of one 2D/3D FFT-conv call with a shared fp32
    filter [C, *K] and a shortcut [C] in the I/O dtype (same accounting as
    :func:`algorithmic_bytes_causal1d`).  Config 4 forward: 427,819,776 B;
    config 5 forward + backward: 1,073,742,592 B."""
    E = B * C * math.prod(S)
    KK = C * math.prod(K)
    if phase == "fwd":
        return E * 2 * itemsize + KK * 4 + C * itemsize
    if phase == "bwd":
        return E * 3 * itemsize + KK * 8 + 2 * C * itemsize
    if phase == "fwd+bwd":
        return algorithmic_bytes_nd(B, C, S, K, itemsize, "fwd") + algorithmic_bytes_nd(B, C, S, K, itemsize, "bwd")
    raise ValueError(phase)


def algorithmic_bytes_gated(B: int, H: int, L: int, K: int, itemsize: int) -> int:
    """Compulsory HBM bytes of one gated causal FFT-conv forward + backward (Hyena layer's
    ``(conv(q act1(k)) + s z) act2(v)``): forward reads q, k, v and writes y and the kept
    y1 (5 tensors); backward reads g, q, k, v, y1 and writes dq, dk, dv (8 tensors); the fp32
    filter is read by both and its gradient written once; shortcut read twice, its
    gradient written once."""
    E = B * H * L
    return E * itemsize * 13 + H * K * 4 * 3 + H * itemsize * 3
