"""CPU restatement of the reference circular FFT convolution -- TEST INFRASTRUCTURE ONLY.

* :func:`circular_fftconv_torch` follows nvsubquadratic/ops/circular_fftconv.py
  step for step in float32 CPU torch (1D :310-404, 2D and 3D the same steps over
  2 or 3 axes): cast to fp32, ``rfftn`` of x and of the kernel at the input's
  own sizes (no padding; the kernel is zero-extended), multiply by the
  phase ramp of the integer shift ``-((K_d - 1) // 2)`` per axis
  (``_PhaseRampCache*.get``: ``exp(-2 pi i sum_d shift_d f_d)`` with
  ``fftfreq`` / ``rfftfreq``), ``irfftn``, cast to ``x.dtype``, then
  ``+ shortcut * x``.  Autograd-capable: its gradients are the reference's.
* :func:`circular_conv_direct_np` is the brute-force float64 circular
  convolution the reference's own tests compare against
  (tests/ops/test_circular_fftconv.py:69-105: circular padding K//2 left,
  K - 1 - K//2 right, flipped kernel, grouped conv), written out as
  ``y[n] = sum_j k[j] x[(n + (K - 1)//2 - j) mod S]`` per axis.  It pins the
  FFT restatement (tests/test_oracle_circular.py) with no FFT involved.
* :func:`mixed_fftconv_torch` follows nvsubquadratic/ops/mixed_fftconv.py
  (``_mixed_recipe`` :295-343, ``_mixed_fftconv_nd_fp32_bhl`` :504-628): per
  axis FFT length N_d (periodic) or min(N_d + (K_d+1)//2, 2 N_d) (zero), the
  ramp of shift -((K_d-1)//2) on periodic axes only, crop [K_d//2, K_d//2 + N_d)
  on zero axes.  :func:`mixed_conv_direct_np` is its float64 brute force:
  ``y[n] = sum_j k[j] x[n + c_d - j]`` with c_d = (K_d-1)//2 and the index taken
  mod N_d on periodic axes, c_d = K_d//2 and x = 0 outside [0, N_d) on zero axes.
"""

from __future__ import annotations

import itertools
import math

import numpy as np
import torch


def circular_fftconv_torch(x: torch.Tensor, kernel: torch.Tensor, shortcut: torch.Tensor | None = None,
                           compute_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """x ``[B, H, *S]`` (1 to 3 spatial axes), kernel ``[1|B, H, *K]`` (K_d <= S_d).

    ``compute_dtype=torch.float32`` is the reference's arithmetic, phase ramp
    included: its float32 angles ``2 pi c f`` (up to ``pi (K-1)/2``) carry an
    absolute error of about ulp(pi K / 2), i.e. ~1e-4 relative at K ~ 4096.
    ``torch.float64`` gives the exact-math result the GPU parity tests use.
    """
    nd = x.dim() - 2
    S = list(x.shape[2:])
    K = list(kernel.shape[2:])
    dims = tuple(range(2, 2 + nd))
    xf = torch.fft.rfftn(x.to(compute_dtype), s=S, dim=dims)
    kf = torch.fft.rfftn(kernel.to(compute_dtype), s=S, dim=dims)
    # phase ramp of the shift -((K_d - 1) // 2) along every axis (circular_fftconv.py:_PhaseRampCache*)
    phases = torch.zeros([S[d] if d < nd - 1 else S[d] // 2 + 1 for d in range(nd)], dtype=compute_dtype)
    for d in range(nd):
        f = (torch.fft.rfftfreq if d == nd - 1 else torch.fft.fftfreq)(S[d], dtype=compute_dtype)
        shape = [1] * nd
        shape[d] = -1
        phases = phases + (-2.0 * math.pi * -((K[d] - 1) // 2)) * f.reshape(shape)
    kf = kf * torch.complex(torch.cos(phases), torch.sin(phases))
    y = torch.fft.irfftn(xf * kf, s=S, dim=dims).to(x.dtype)
    if shortcut is not None:
        y = y + shortcut.to(x.dtype).reshape([1, -1] + [1] * nd) * x
    return y


def circular_conv_direct_np(x, kernel, shortcut=None) -> np.ndarray:
    """float64 brute force: y[b,h,n] = sum_j k[b|0,h,j] x[b,h,(n + c - j) mod S] per axis, c = (K-1)//2."""
    x = np.asarray(x, dtype=np.float64)
    k = np.asarray(kernel, dtype=np.float64)
    nd = x.ndim - 2
    S = x.shape[2:]
    K = k.shape[2:]
    c = [(kd - 1) // 2 for kd in K]
    y = np.zeros_like(x)
    for j in itertools.product(*[range(kd) for kd in K]):
        # x[(n + c - j) mod S] = roll(x, shift = j - c)
        shifted = np.roll(x, shift=[j[d] - c[d] for d in range(nd)], axis=tuple(range(2, 2 + nd)))
        w = k[(slice(None), slice(None)) + tuple(j)]  # [1|B, H]
        y += w.reshape(w.shape + (1,) * nd) * shifted
    if shortcut is not None:
        y += np.asarray(shortcut, dtype=np.float64).reshape([1, -1] + [1] * nd) * x
    return y


def mixed_fftconv_torch(x: torch.Tensor, kernel: torch.Tensor, periodic, shortcut: torch.Tensor | None = None,
                        compute_dtype: torch.dtype = torch.float32):
    """x ``[B, H, *S]``, kernel ``[1|B, H, *K]``, periodic: one bool per spatial axis (compute_dtype as above)."""
    nd = x.dim() - 2
    S = list(x.shape[2:])
    K = list(kernel.shape[2:])
    dims = tuple(range(2, 2 + nd))
    F = [S[d] if periodic[d] else min(S[d] + (K[d] + 1) // 2, 2 * S[d]) for d in range(nd)]
    xf = torch.fft.rfftn(x.to(compute_dtype), s=F, dim=dims)
    kf = torch.fft.rfftn(kernel.to(compute_dtype), s=F, dim=dims)
    phases = torch.zeros([F[d] if d < nd - 1 else F[d] // 2 + 1 for d in range(nd)], dtype=compute_dtype)
    for d in range(nd):
        if not periodic[d]:
            continue
        f = (torch.fft.rfftfreq if d == nd - 1 else torch.fft.fftfreq)(F[d], dtype=compute_dtype)
        shape = [1] * nd
        shape[d] = -1
        phases = phases + (-2.0 * math.pi * -((K[d] - 1) // 2)) * f.reshape(shape)
    kf = kf * torch.complex(torch.cos(phases), torch.sin(phases))
    y = torch.fft.irfftn(xf * kf, s=F, dim=dims)
    crop = tuple(slice(0, S[d]) if periodic[d] else slice(K[d] // 2, K[d] // 2 + S[d]) for d in range(nd))
    y = y[(slice(None), slice(None)) + crop].to(x.dtype)
    if shortcut is not None:
        y = y + shortcut.to(x.dtype).reshape([1, -1] + [1] * nd) * x
    return y


def _shift_axis(a: np.ndarray, shift: int, axis: int, periodic: bool) -> np.ndarray:
    """out[n] = a[n - shift] along `axis`: wrapped (periodic) or zero-filled."""
    if periodic:
        return np.roll(a, shift, axis=axis)
    out = np.zeros_like(a)
    n = a.shape[axis]
    if abs(shift) >= n:
        return out
    src = [slice(None)] * a.ndim
    dst = [slice(None)] * a.ndim
    if shift >= 0:
        src[axis], dst[axis] = slice(0, n - shift), slice(shift, n)
    else:
        src[axis], dst[axis] = slice(-shift, n), slice(0, n + shift)
    out[tuple(dst)] = a[tuple(src)]
    return out


def mixed_conv_direct_np(x, kernel, periodic, shortcut=None) -> np.ndarray:
    """float64 brute force of the mixed-boundary "same" convolution (see the module docstring)."""
    x = np.asarray(x, dtype=np.float64)
    k = np.asarray(kernel, dtype=np.float64)
    nd = x.ndim - 2
    K = k.shape[2:]
    c = [(K[d] - 1) // 2 if periodic[d] else K[d] // 2 for d in range(nd)]
    y = np.zeros_like(x)
    for j in itertools.product(*[range(kd) for kd in K]):
        shifted = x
        for d in range(nd):
            shifted = _shift_axis(shifted, j[d] - c[d], 2 + d, bool(periodic[d]))
        w = k[(slice(None), slice(None)) + tuple(j)]
        y += w.reshape(w.shape + (1,) * nd) * shifted
    if shortcut is not None:
        y += np.asarray(shortcut, dtype=np.float64).reshape([1, -1] + [1] * nd) * x
    return y
