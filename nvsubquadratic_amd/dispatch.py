"""``fft_backend="hip"`` selection, mirroring CKConvND's backend dispatch.

The reference chooses its FFT-conv functions in ``CKConvND.__init__``
(``nvsubquadratic/modules/ckconv_nd.py:628-630`` for the backend assert,
``:700-724`` for the subq_ops constraints, ``:796-871`` for the selection).  This
module provides the ``"hip"`` branch with the same contract:

* :data:`FFT_BACKENDS` extends the accepted set to ``("torch_fft", "subq_ops", "hip")``;
* :func:`validate_hip_backend` raises the same exception types the reference
  raises for unsupported combinations (1D must be causal; 2D/3D must be
  zero-padded and non-causal; no per-axis / circular padding);
* :func:`hip_fftconv_fns` returns ``(fftconv_fn, fftconv_fn_bhl_input)``, the
  pair CKConvND stores and calls in ``apply_convolution``
  (``ckconv_nd.py:1054-1062``).

The 2D/3D families are exposed once their kernels are built (see
``fftconv_hip.fftconv2d_bhl`` / ``fftconv3d_bhl``).
"""

from __future__ import annotations

from collections.abc import Sequence

from . import fftconv_hip as F


__all__ = ["FFT_BACKENDS", "hip_fftconv_fns", "validate_fft_backend", "validate_hip_backend"]

FFT_BACKENDS = ("torch_fft", "subq_ops", "hip")


def validate_fft_backend(fft_backend: str) -> None:
    """Backend name check (``ckconv_nd.py:628-630`` with ``"hip"`` added)."""
    assert fft_backend in FFT_BACKENDS, (
        f"Invalid fft_backend: {fft_backend!r}. Must be 'torch_fft', 'subq_ops' or 'hip'."
    )


def _is_tuple_mode(fft_padding) -> bool:
    return isinstance(fft_padding, Sequence) and not isinstance(fft_padding, (str, bytes))


def validate_hip_backend(data_dim: int, is_causal: bool, fft_padding) -> None:
    """Constraint block of the hip backend (same checks as ``ckconv_nd.py:700-724``).

    1D requires ``is_causal=True``; 2D and 3D require ``is_causal=False`` and
    ``fft_padding == "zero"``; per-axis padding lists are rejected.
    """
    if _is_tuple_mode(fft_padding):
        raise ValueError(
            "fft_backend='hip' does not support a per-axis fft_padding. "
            "The HIP kernels implement zero-padded conv only. "
            "Use fft_backend='torch_fft' for mixed boundary conditions."
        )
    if data_dim == 1:
        assert is_causal, (
            "fft_backend='hip' on 1D requires is_causal=True "
            "(no non-causal 1D HIP kernel is wired). Got is_causal=False."
        )
    elif data_dim in (2, 3):
        assert not is_causal, (
            f"fft_backend='hip' on {data_dim}D does not support causal convolutions (causal is 1D only)."
        )
        assert fft_padding == "zero", (
            f"fft_backend='hip' on {data_dim}D only supports zero-padded convolutions. "
            f"Got fft_padding='{fft_padding}'."
        )
    else:
        raise AssertionError(f"fft_backend='hip' only supports data_dim in (1, 2, 3). Got data_dim={data_dim}.")


def hip_fftconv_fns(data_dim: int, is_causal: bool, fft_padding="zero", use_chunked_fftconv: bool = False):
    """Return ``(fftconv_fn, fftconv_fn_bhl_input)`` for the hip backend.

    ``fftconv_fn`` takes BLH input (``*_bhl_w_reshape``), ``fftconv_fn_bhl_input``
    takes BHL input, exactly as the reference's tables
    (``ckconv_nd.py:202-232``) and its subq_ops branch (``:797-831``).
    """
    validate_hip_backend(data_dim, is_causal, fft_padding)
    if data_dim == 1:
        if use_chunked_fftconv:
            return F.causal_fftconv1d_bhl_w_reshape_chunked, F.causal_fftconv1d_bhl_chunked
        return F.causal_fftconv1d_bhl_w_reshape, F.causal_fftconv1d_bhl
    if data_dim == 2:
        if use_chunked_fftconv:
            return F.fftconv2d_bhl_w_reshape_chunked, F.fftconv2d_bhl_chunked
        return F.fftconv2d_bhl_w_reshape, F.fftconv2d_bhl
    if use_chunked_fftconv:
        return F.fftconv3d_bhl_w_reshape_chunked, F.fftconv3d_bhl_chunked
    return F.fftconv3d_bhl_w_reshape, F.fftconv3d_bhl
