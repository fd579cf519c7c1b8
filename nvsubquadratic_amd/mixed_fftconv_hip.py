r"""HIP mixed-boundary FFT convolution with the ``nvsubquadratic.ops.mixed_fftconv`` signatures.

Reference: ``nvsubquadratic/ops/mixed_fftconv.py`` (torch.fft only).  Each
spatial axis is either periodic (circular conv, FFT length ``N_d``, output
rolled by ``-((K_d - 1) // 2)``, ``K_d <= N_d``) or zero-padded "same"
(linear conv cropped at ``K_d // 2``, ``K_d <= 2 N_d``) -- the recipe of
``_mixed_recipe`` (``mixed_fftconv.py:295-343``).  Uniform ``periodic`` tuples
route to the circular or zero-padded op exactly as the reference's
``_dispatch_legacy_if_uniform`` (``:445-501``).

How: one call of the HIP N-d engine with the per-axis mask
(``nsq_mixed_fftconv_nd_*``; bit d = axis d periodic).  1D runs the fused 1D
kernels with the output shift on the filter's spectrum
(``nsq_mixed_fftconv1d_*``): ``periodic=(True,)`` the circular op,
``periodic=(False,)`` the zero-padded one (``fftconv_hip.fftconv1d_bhl``).
Periodic axes whose length is not a power of two run on the periodic
extension of x as zero-padded axes
(:func:`circular_fftconv_hip.periodic_by_extension`).
"""

from __future__ import annotations

from collections.abc import Sequence

import torch
from einops import rearrange

from . import circular_fftconv_hip as _circ
from . import fftconv_hip as _zero


__all__ = [
    "mixed_fftconv1d_fp32_bhl",
    "mixed_fftconv1d_fp32_bhl_chunked",
    "mixed_fftconv1d_fp32_bhl_w_reshape",
    "mixed_fftconv1d_fp32_bhl_w_reshape_chunked",
    "mixed_fftconv2d_fp32_bhl",
    "mixed_fftconv2d_fp32_bhl_chunked",
    "mixed_fftconv2d_fp32_bhl_w_reshape",
    "mixed_fftconv2d_fp32_bhl_w_reshape_chunked",
    "mixed_fftconv3d_fp32_bhl",
    "mixed_fftconv3d_fp32_bhl_chunked",
    "mixed_fftconv3d_fp32_bhl_w_reshape",
    "mixed_fftconv3d_fp32_bhl_w_reshape_chunked",
    "periodic_mask",
]

_DEFAULT_MIXED_CHUNK_SIZE = 128
_RESHAPE = {
    1: ("b l h -> b h l", "b k h -> b h k", "b h l -> b l h"),
    2: ("b x y h -> b h x y", "b kx ky h -> b h kx ky", "b h x y -> b x y h"),
    3: ("b x y z h -> b h x y z", "b kx ky kz h -> b h kx ky kz", "b h x y z -> b x y z h"),
}


def _normalize_periodic(periodic: Sequence[bool], data_dim: int) -> tuple[bool, ...]:
    """``mixed_fftconv.py:420-442``."""
    periodic_t = tuple(bool(p) for p in periodic)
    assert len(periodic_t) == data_dim, (
        f"periodic must have length {data_dim} (data_dim), got length {len(periodic_t)}"
    )
    return periodic_t


def periodic_mask(periodic: Sequence[bool]) -> int:
    """Bit d set = axis d periodic (the ``periodic`` argument of ``nsq_mixed_fftconv_nd_*``)."""
    return sum(1 << d for d, p in enumerate(periodic) if p)


def _mixed_core(x, kernel, periodic_t, shortcut, use_phase_shift, data_dim):
    """Shape checks and dispatch of ``_mixed_fftconv_nd_fp32_bhl`` (``mixed_fftconv.py:504-628``)."""
    assert x.ndim == 2 + data_dim, f"Expected {2 + data_dim}D input, got {x.ndim}D"
    assert kernel.ndim == 2 + data_dim, f"Expected {2 + data_dim}D kernel, got {kernel.ndim}D"
    B, H = x.shape[:2]
    assert kernel.shape[0] in (1, B), (
        f"Leading kernel dim must be 1 or batch_size ({B}). Got kernel.shape={tuple(kernel.shape)}."
    )
    assert kernel.shape[1] == H, f"Kernel hidden dim ({kernel.shape[1]}) must equal input hidden dim ({H})."
    for d, (N, K, is_periodic) in enumerate(zip(x.shape[2:], kernel.shape[2:], periodic_t)):
        if is_periodic:
            assert K <= N, f"K must be <= N on periodic axis {d}: K={K}, N={N}."
        else:
            assert K <= 2 * N, f"K must be <= 2*N on non-periodic axis {d}: K={K}, N={N}."
    if all(periodic_t):
        fn = (_circ.circular_fftconv1d_fp32_bhl, _circ.circular_fftconv2d_fp32_bhl,
              _circ.circular_fftconv3d_fp32_bhl)[data_dim - 1]
        return fn(x, kernel, shortcut, use_phase_shift=use_phase_shift)
    if not any(periodic_t):
        return (_zero.fftconv1d_bhl, _zero.fftconv2d_bhl, _zero.fftconv3d_bhl)[data_dim - 1](x, kernel, shortcut)
    if shortcut is not None:
        assert shortcut.dtype == x.dtype, f"shortcut.dtype ({shortcut.dtype}) must match x.dtype ({x.dtype})"
        assert shortcut.shape == (H,), f"Expected shortcut shape ({H},), got {tuple(shortcut.shape)}"
    if _circ.needs_extension(x.shape[2:], periodic_t):
        return _circ.periodic_by_extension(x, kernel, shortcut, periodic_t)
    return _zero._nd_core(x, kernel, shortcut, data_dim, periodic=periodic_mask(periodic_t))


def _chunked(x, kernel, shortcut, chunk_size, fn):
    """``_chunked_along_channels`` (``mixed_fftconv.py:833-874``)."""
    H = x.shape[1]
    if H <= chunk_size:
        return fn(x, kernel, shortcut)
    outs = []
    for start in range(0, H, chunk_size):
        end = min(start + chunk_size, H)
        outs.append(fn(x[:, start:end], kernel[:, start:end], None if shortcut is None else shortcut[start:end]))
    return torch.cat(outs, dim=1)


def _make(data_dim: int):
    def bhl(x: torch.Tensor, kernel: torch.Tensor, periodic: Sequence[bool], shortcut: torch.Tensor | None = None,
            use_phase_shift: bool = True) -> torch.Tensor:
        periodic_t = _normalize_periodic(periodic, data_dim)
        return _mixed_core(x, kernel, periodic_t, shortcut, use_phase_shift, data_dim)

    def bhl_chunked(x, kernel, periodic, shortcut=None, use_phase_shift=True, chunk_size=None):
        chunk = chunk_size if chunk_size is not None else _DEFAULT_MIXED_CHUNK_SIZE
        periodic_t = _normalize_periodic(periodic, data_dim)
        return _chunked(x, kernel, shortcut, chunk,
                        lambda xc, kc, sc: _mixed_core(xc, kc, periodic_t, sc, use_phase_shift, data_dim))

    rx, rk, ry = _RESHAPE[data_dim]

    def w_reshape(x, kernel, periodic, shortcut=None, use_phase_shift=True):
        return rearrange(bhl(rearrange(x, rx), rearrange(kernel, rk), periodic, shortcut, use_phase_shift), ry)

    def w_reshape_chunked(x, kernel, periodic, shortcut=None, use_phase_shift=True, chunk_size=None):
        y = bhl_chunked(rearrange(x, rx), rearrange(kernel, rk), periodic, shortcut, use_phase_shift, chunk_size)
        return rearrange(y, ry)

    # definition lines in mixed_fftconv.py: (bhl, chunked, w_reshape, w_reshape_chunked)
    lines = {1: (631, 877, 731, 989), 2: (663, 914, 762, 1028), 3: (700, 949, 792, 1065)}[data_dim]
    for f, suffix, line in zip((bhl, bhl_chunked, w_reshape, w_reshape_chunked),
                               ("", "_chunked", "_w_reshape", "_w_reshape_chunked"), lines):
        f.__name__ = f.__qualname__ = f"mixed_fftconv{data_dim}d_fp32_bhl{suffix}"
        f.__doc__ = (f"{data_dim}D mixed-BC FFT conv on the HIP N-d engine; same signature and results as "
                     f"``nvsubquadratic.ops.mixed_fftconv.{f.__name__}`` (mixed_fftconv.py:{line}).")
    return bhl, bhl_chunked, w_reshape, w_reshape_chunked


(mixed_fftconv1d_fp32_bhl, mixed_fftconv1d_fp32_bhl_chunked, mixed_fftconv1d_fp32_bhl_w_reshape,
 mixed_fftconv1d_fp32_bhl_w_reshape_chunked) = _make(1)
(mixed_fftconv2d_fp32_bhl, mixed_fftconv2d_fp32_bhl_chunked, mixed_fftconv2d_fp32_bhl_w_reshape,
 mixed_fftconv2d_fp32_bhl_w_reshape_chunked) = _make(2)
(mixed_fftconv3d_fp32_bhl, mixed_fftconv3d_fp32_bhl_chunked, mixed_fftconv3d_fp32_bhl_w_reshape,
 mixed_fftconv3d_fp32_bhl_w_reshape_chunked) = _make(3)
