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
    "algorithmic_bytes_causal1d",
    "causal1d_case",
    "causal1d_case_fast",
    "decaying_filter_1d",
    "fft_flops_causal1d",
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
