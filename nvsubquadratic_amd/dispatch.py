"""``fft_backend="hip"`` selection, mirroring CKConvND's backend dispatch.

The reference chooses its FFT-conv functions in ``CKConvND.__init__``
(``nvsubquadratic/modules/ckconv_nd.py:628-630`` for the backend assert,
``:690-724`` for the circular and subq_ops constraints, ``:796-871`` for the
selection, ``:280-375`` ``_resolve_periodic`` for per-axis padding lists and
``:378-403`` ``_wrap_mixed_op``).  This module provides the ``"hip"`` branch
with the same contract:

* :data:`FFT_BACKENDS` extends the accepted set to ``("torch_fft", "subq_ops", "hip")``;
* :func:`validate_hip_backend` raises the reference's exception types for the
  combinations the HIP kernels do not cover: 2D/3D must be non-causal (1D
  takes causal, zero, circular or a per-axis list);
* :func:`hip_fftconv_fns` returns ``(fftconv_fn, fftconv_fn_bhl_input)``, the
  pair CKConvND stores and calls in ``apply_convolution``
  (``ckconv_nd.py:1054-1062``): the causal / zero-padded ops of
  :mod:`.fftconv_hip`, the circular ops of :mod:`.circular_fftconv_hip`
  (``fft_padding="circular"``, the reference's ``FFT_FUNCTIONS["circular"]``
  table, ``:201-217``) or, for a per-axis list, the mixed ops of
  :mod:`.mixed_fftconv_hip` with ``periodic`` bound (``:238-248``, ``:828-845``).
"""

from __future__ import annotations

from collections.abc import Sequence

from . import circular_fftconv_hip as C
from . import fftconv_hip as F
from . import mixed_fftconv_hip as M


__all__ = ["FFT_BACKENDS", "hip_fftconv_fns", "resolve_periodic", "validate_fft_backend", "validate_hip_backend"]

FFT_BACKENDS = ("torch_fft", "subq_ops", "hip")


def validate_fft_backend(fft_backend: str) -> None:
    """Backend name check (``ckconv_nd.py:628-630`` with ``"hip"`` added)."""
    assert fft_backend in FFT_BACKENDS, (
        f"Invalid fft_backend: {fft_backend!r}. Must be 'torch_fft', 'subq_ops' or 'hip'."
    )


def _is_tuple_mode(fft_padding) -> bool:
    return isinstance(fft_padding, Sequence) and not isinstance(fft_padding, (str, bytes))


_PADDING_MODE_TO_PERIODIC = {"zero": False, "circular": True}


def resolve_periodic(fft_padding, data_dim: int) -> tuple[bool, ...]:
    """Per-axis periodic flags of ``fft_padding`` (``ckconv_nd.py:280-375``, same errors)."""
    if isinstance(fft_padding, bool):
        raise ValueError(
            "fft_padding=True/False is not a valid input. Use 'zero' (all axes zero-padded), 'circular' "
            "(all axes periodic), or a per-axis list of mode strings such as ['circular', 'zero'].")

    def parse(mode: str) -> bool:
        m = mode.strip().lower()
        if m not in _PADDING_MODE_TO_PERIODIC:
            raise ValueError(f"Invalid padding mode {mode!r}. Must be one of {sorted(_PADDING_MODE_TO_PERIODIC)}.")
        return _PADDING_MODE_TO_PERIODIC[m]

    if isinstance(fft_padding, str):
        if "," in fft_padding:
            raise ValueError(
                f"fft_padding does not accept comma-separated strings (got {fft_padding!r}). For per-axis "
                f"modes use a list, e.g. ['circular', 'zero'].")
        return (parse(fft_padding),) * data_dim
    if _is_tuple_mode(fft_padding):
        items = list(fft_padding)
        if any(isinstance(item, bool) for item in items):
            raise ValueError(
                "fft_padding no longer accepts a sequence of booleans (e.g. (True, False)); use mode strings "
                "instead: ['circular', 'zero'].")
        if not all(isinstance(item, str) for item in items):
            raise ValueError(f"fft_padding sequence must contain only padding-mode strings. Got: {fft_padding!r}.")
        if len(items) != data_dim:
            raise ValueError(
                f"fft_padding sequence must have length data_dim={data_dim}, got length {len(items)}: "
                f"{fft_padding!r}.")
        return tuple(parse(item) for item in items)
    raise ValueError(
        f"fft_padding must be a single mode string ('zero' / 'circular') or a sequence of mode strings "
        f"(one per spatial axis). Got {fft_padding!r} (type {type(fft_padding).__name__}).")


def validate_hip_backend(data_dim: int, is_causal: bool, fft_padding, use_chunked_fftconv: bool = False) -> None:
    """Constraint block of the hip backend (the checks of ``ckconv_nd.py:690-724`` for what HIP covers).

    1D: causal, or non-causal with ``"zero"``, ``"circular"`` or a per-axis list;
    2D and 3D: ``is_causal=False`` with ``"zero"``, ``"circular"`` or a per-axis
    list.  ``"circular"`` (string form) takes no chunked variant, as in the
    reference (``:695-699``).
    """
    if data_dim not in (1, 2, 3):
        raise AssertionError(f"fft_backend='hip' only supports data_dim in (1, 2, 3). Got data_dim={data_dim}.")
    periodic = resolve_periodic(fft_padding, data_dim)
    if not _is_tuple_mode(fft_padding) and fft_padding.strip().lower() == "circular":
        assert not use_chunked_fftconv, (
            "use_chunked_fftconv=True is not supported with fft_padding='circular'. Chunked FFT convolutions "
            "are only implemented for 'zero' padding (and 'causal' 1D).")
    if data_dim == 1:
        return
    assert not is_causal, (
        f"fft_backend='hip' on {data_dim}D does not support causal convolutions (causal is 1D only)."
    )


def _bind_periodic(op, periodic: tuple[bool, ...]):
    """``_wrap_mixed_op`` (``ckconv_nd.py:378-403``): fix ``periodic`` so the op is called as ``fn(x, k, s)``."""

    def fn(x, kernel, shortcut=None):
        return op(x, kernel, periodic, shortcut)

    fn.__name__ = op.__name__
    fn.__doc__ = op.__doc__
    fn.periodic = periodic
    fn.op = op
    return fn


def hip_fftconv_fns(data_dim: int, is_causal: bool, fft_padding="zero", use_chunked_fftconv: bool = False):
    """Return ``(fftconv_fn, fftconv_fn_bhl_input)`` for the hip backend.

    ``fftconv_fn`` takes BLH input (``*_bhl_w_reshape``), ``fftconv_fn_bhl_input``
    takes BHL input, exactly as the reference's tables
    (``ckconv_nd.py:202-248``) and its selection branches (``:797-871``).
    """
    validate_hip_backend(data_dim, is_causal, fft_padding, use_chunked_fftconv)
    if data_dim == 1 and is_causal:
        if use_chunked_fftconv:
            return F.causal_fftconv1d_bhl_w_reshape_chunked, F.causal_fftconv1d_bhl_chunked
        return F.causal_fftconv1d_bhl_w_reshape, F.causal_fftconv1d_bhl
    periodic = resolve_periodic(fft_padding, data_dim)
    if _is_tuple_mode(fft_padding):
        mixed = {
            (1, False): (M.mixed_fftconv1d_fp32_bhl_w_reshape, M.mixed_fftconv1d_fp32_bhl),
            (2, False): (M.mixed_fftconv2d_fp32_bhl_w_reshape, M.mixed_fftconv2d_fp32_bhl),
            (3, False): (M.mixed_fftconv3d_fp32_bhl_w_reshape, M.mixed_fftconv3d_fp32_bhl),
            (1, True): (M.mixed_fftconv1d_fp32_bhl_w_reshape_chunked, M.mixed_fftconv1d_fp32_bhl_chunked),
            (2, True): (M.mixed_fftconv2d_fp32_bhl_w_reshape_chunked, M.mixed_fftconv2d_fp32_bhl_chunked),
            (3, True): (M.mixed_fftconv3d_fp32_bhl_w_reshape_chunked, M.mixed_fftconv3d_fp32_bhl_chunked),
        }[(data_dim, bool(use_chunked_fftconv))]
        return _bind_periodic(mixed[0], periodic), _bind_periodic(mixed[1], periodic)
    if all(periodic):
        return {
            1: (C.circular_fftconv1d_fp32_bhl_w_reshape, C.circular_fftconv1d_fp32_bhl),
            2: (C.circular_fftconv2d_fp32_bhl_w_reshape, C.circular_fftconv2d_fp32_bhl),
            3: (C.circular_fftconv3d_fp32_bhl_w_reshape, C.circular_fftconv3d_fp32_bhl),
        }[data_dim]
    if data_dim == 1:
        if use_chunked_fftconv:
            return F.fftconv1d_bhl_w_reshape_chunked, F.fftconv1d_bhl_chunked
        return F.fftconv1d_bhl_w_reshape, F.fftconv1d_bhl
    if data_dim == 2:
        if use_chunked_fftconv:
            return F.fftconv2d_bhl_w_reshape_chunked, F.fftconv2d_bhl_chunked
        return F.fftconv2d_bhl_w_reshape, F.fftconv2d_bhl
    if use_chunked_fftconv:
        return F.fftconv3d_bhl_w_reshape_chunked, F.fftconv3d_bhl_chunked
    return F.fftconv3d_bhl_w_reshape, F.fftconv3d_bhl
