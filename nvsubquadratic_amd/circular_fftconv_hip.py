r"""HIP circular (periodic) FFT convolution with the ``nvsubquadratic.ops.circular_fftconv`` signatures.

Reference: ``nvsubquadratic/ops/circular_fftconv.py`` (torch.fft only, no
native kernel).  Per axis of length ``S_d`` with a kernel of ``K_d <= S_d``
taps the output is the circular convolution aligned to "same":

    y[n] = sum_j k[j] x[(n + (K_d - 1) // 2 - j) mod S_d]

(the reference's ``rfftn(x) * rfftn(k) * phase_ramp`` with shift
``-((K_d - 1) // 2)``, ``circular_fftconv.py:310-404``), cast to ``x.dtype``,
then ``+ shortcut * x``.

How: the 2D / 3D calls run the HIP N-d engine with every axis periodic
(``nsq_mixed_fftconv_nd_*``): FFT length ``S_d`` (no padding), the shift as a
ramp folded into the filter values of the product pass, no crop.  The 1D call
runs ``nsq_mixed_fftconv1d_*`` with ``periodic=1``: the fused 1D kernels at FFT
length ``L`` with the ramp on the filter's spectrum, or beyond 16384 the 4-step
plan on a rolled copy of x (g in the backward).  ``use_phase_shift`` is accepted for
signature parity; both of the reference's branches give the same result and
the kernels always apply the shift in the frequency domain.

Sizes: power-of-two periodic lengths run as above (2D / 3D: up to 1024 per
axis; 1D: up to 2^24, the fused kernels up to 16384 and the 4-step plan
beyond; lengths below 16 on their periodic extension at FFT length 16).  A
periodic axis of any other length S runs as a zero-padded "same" axis on the
periodic extension of x (:func:`periodic_by_extension`): the circular sums
are exactly the linear ones over S + K - 1 extended samples, so the result is
the reference's at FFT length pow2(S + K - 1 + ceil(K/2)) (2D / 3D: up to
1024 per axis).  Sizes beyond that raise ``NotImplementedError`` (the product
has no CPU fallback).
"""

from __future__ import annotations

import torch
from einops import rearrange

from . import _lib
from .fftconv_hip import _nd_core, fftconv1d_bhl, shifted_fftconv1d


__all__ = [
    "circular_fftconv1d_fp32_bhl",
    "circular_fftconv1d_fp32_bhl_w_reshape",
    "circular_fftconv2d_fp32_bhl",
    "circular_fftconv2d_fp32_bhl_w_reshape",
    "circular_fftconv3d_fp32_bhl",
    "circular_fftconv3d_fp32_bhl_w_reshape",
    "circular_fftconv1d_fwd_raw",
    "circular_fftconv1d_bwd_raw",
]


def _pow2(n: int) -> bool:
    return n > 0 and n & (n - 1) == 0


def needs_extension(shape, periodic) -> bool:
    """True if a periodic axis has a length the power-of-two periodic plans do not take."""
    return any(p and not _pow2(int(n)) for n, p in zip(shape, periodic))


def periodic_by_extension(x: torch.Tensor, kernel: torch.Tensor, shortcut: torch.Tensor | None,
                          periodic) -> torch.Tensor:
    """Mixed / circular conv whose periodic axes include lengths that are not powers of two.

    On such an axis (length S, K <= S taps, c = (K - 1) // 2) the circular "same" output
    ``y[n] = sum_j k[j] x[(n + c - j) mod S]`` equals the zero-padded "same" conv of the periodic
    extension ``xe[t] = x[(t - (K - 1 - c)) mod S]``, t < S + K - 1, read at ``n + c``: every index
    ``n + c + K//2 - j`` it sums over lies in [0, S + K - 1), so no zero padding enters the kept window
    (and the extension wraps at most once, K <= S).  The other axes keep their own mode (power-of-two
    periodic axes stay on the shift-ramp plan).  The extension is a gather (its gradient the
    matching scatter-add, by autograd), the conv is the HIP op, and the shortcut is added afterwards as
    the reference adds it (``y.to(x.dtype) + shortcut * x``, ``mixed_fftconv.py:616-623``).
    """
    nd = x.dim() - 2
    xe = x
    crops = []
    mask = 0
    for d, (n, kk, p) in enumerate(zip(x.shape[2:], kernel.shape[2:], periodic)):
        if p and not _pow2(int(n)):
            c = (kk - 1) // 2
            idx = (torch.arange(n + kk - 1, device=x.device) - (kk - 1 - c)) % n
            xe = xe.index_select(2 + d, idx)
            crops.append(slice(c, c + n))
        else:
            mask |= (1 << d) if p else 0
            crops.append(slice(None))
    if nd == 1:  # the one axis was extended: zero-padded
        y = fftconv1d_bhl(xe, kernel, None)
    else:
        y = _nd_core(xe, kernel, None, nd, periodic=mask)
    y = y[(slice(None), slice(None), *crops)]
    if shortcut is not None:
        y = y + shortcut.view(1, -1, *([1] * nd)) * x
    return y


def _check_common(x: torch.Tensor, kernel: torch.Tensor, shortcut: torch.Tensor | None, nd: int) -> None:
    """Argument checks of the reference (``circular_fftconv.py:363-369, 400-401, 440-447, 539-545``)."""
    B, H = x.shape[:2]
    assert len(kernel.shape) == nd + 2, f"Unexpected kernel shape: {kernel.shape}."
    assert kernel.shape[0] in (1, B), (
        f"Leading dimension must be 1 or batch_size ({B}). Got kernel.shape={kernel.shape}."
    )
    assert kernel.shape[1] == H, "Input and kernel must have the same number of channels (H)."
    for d in range(nd):
        assert kernel.shape[2 + d] <= x.shape[2 + d], (
            f"Kernel must be <= input along each axis. Got K={tuple(kernel.shape[2:])}, S={tuple(x.shape[2:])}."
        )
    if shortcut is not None:
        assert shortcut.dtype == x.dtype, f"shortcut.dtype ({shortcut.dtype}) must match x.dtype ({x.dtype})"
        assert shortcut.shape == (H,)


# ---------------------------------------------------------------------------
# 1D: fused kernels at FFT length L
# ---------------------------------------------------------------------------
def circular_fftconv1d_fwd_raw(x, k, s, y, kbatch: int):
    """Launch the 1D circular forward: x/y ``[B, H, L]``, k float32 ``[kbatch*H, K]``, s ``[H]`` or None."""
    lib = _lib.get_lib()
    _lib.check_device(x)
    B, H, L = x.shape
    _lib.check(lib.nsq_circular_fftconv1d_fwd(
        x.data_ptr(), k.data_ptr(), _lib.ptr(s), y.data_ptr(), _lib.dtype_code(x.dtype), B, H, L, k.shape[-1],
        kbatch, _lib.stream_ptr(x.device)))
    return y


def circular_fftconv1d_bwd_raw(g, x, k, s, gx, gk, gs, kbatch: int):
    """Launch the 1D circular backward (gk ``[kbatch*H, K]``, gs ``[kbatch*H]`` partials or None)."""
    lib = _lib.get_lib()
    _lib.check_device(x)
    B, H, L = x.shape
    _lib.check(lib.nsq_circular_fftconv1d_bwd(
        g.data_ptr(), x.data_ptr(), k.data_ptr(), _lib.ptr(s), gx.data_ptr(), gk.data_ptr(), _lib.ptr(gs),
        _lib.dtype_code(x.dtype), B, H, L, k.shape[-1], kbatch, _lib.stream_ptr(x.device)))


def circular_fftconv1d_fp32_bhl(
    x: torch.Tensor,
    kernel: torch.Tensor,
    shortcut: torch.Tensor | None = None,
    use_phase_shift: bool = True,
) -> torch.Tensor:
    """1D circular conv, BHL ``[B, H, L]``, kernel ``[1|B, H, K]`` (``circular_fftconv.py:310-404``)."""
    del use_phase_shift  # same result either way (see module docstring)
    _check_common(x, kernel, shortcut, 1)
    if needs_extension(x.shape[2:], (True,)):
        return periodic_by_extension(x, kernel, shortcut, (True,))
    return shifted_fftconv1d(x, kernel, shortcut, 1)


def circular_fftconv2d_fp32_bhl(
    x: torch.Tensor,
    kernel: torch.Tensor,
    shortcut: torch.Tensor | None = None,
    use_phase_shift: bool = True,
) -> torch.Tensor:
    """2D circular conv, ``[B, H, X, Y]``, kernel ``[1|B, H, Kx, Ky]`` (``circular_fftconv.py:406-483``)."""
    del use_phase_shift
    assert x.ndim == 4, f"x must be [B, H, X, Y]; got {tuple(x.shape)}"
    _check_common(x, kernel, shortcut, 2)
    if needs_extension(x.shape[2:], (True, True)):
        return periodic_by_extension(x, kernel, shortcut, (True, True))
    return _nd_core(x, kernel, shortcut, 2, periodic=0b11)


def circular_fftconv3d_fp32_bhl(
    x: torch.Tensor,
    kernel: torch.Tensor,
    shortcut: torch.Tensor | None = None,
    use_phase_shift: bool = True,
) -> torch.Tensor:
    """3D circular conv, ``[B, H, X, Y, Z]``, kernel ``[1|B, H, Kx, Ky, Kz]`` (``circular_fftconv.py:486-569``)."""
    del use_phase_shift
    assert x.ndim == 5, f"x must be [B, H, X, Y, Z]; got {tuple(x.shape)}"
    _check_common(x, kernel, shortcut, 3)
    if needs_extension(x.shape[2:], (True, True, True)):
        return periodic_by_extension(x, kernel, shortcut, (True, True, True))
    return _nd_core(x, kernel, shortcut, 3, periodic=0b111)


def circular_fftconv1d_fp32_bhl_w_reshape(x, kernel, shortcut=None, use_phase_shift=True):
    """BLH ``[B, L, H]`` input, kernel ``[1|B, K, H]`` (``circular_fftconv.py:585-607``)."""
    y = circular_fftconv1d_fp32_bhl(rearrange(x, "b l h -> b h l"), rearrange(kernel, "b k h -> b h k"), shortcut,
                                    use_phase_shift)
    return rearrange(y, "b h l -> b l h")


def circular_fftconv2d_fp32_bhl_w_reshape(x, kernel, shortcut=None, use_phase_shift=True):
    """BLH ``[B, X, Y, H]`` input (``circular_fftconv.py:610-632``)."""
    y = circular_fftconv2d_fp32_bhl(rearrange(x, "b x y h -> b h x y"), rearrange(kernel, "b kx ky h -> b h kx ky"),
                                    shortcut, use_phase_shift)
    return rearrange(y, "b h x y -> b x y h")


def circular_fftconv3d_fp32_bhl_w_reshape(x, kernel, shortcut=None, use_phase_shift=True):
    """BLH ``[B, X, Y, Z, H]`` input (``circular_fftconv.py:635-660``)."""
    y = circular_fftconv3d_fp32_bhl(rearrange(x, "b x y z h -> b h x y z"),
                                    rearrange(kernel, "b kx ky kz h -> b h kx ky kz"), shortcut, use_phase_shift)
    return rearrange(y, "b h x y z -> b x y z h")
