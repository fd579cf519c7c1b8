"""ctypes binding of the gfx950 C-ABI library ``libnsq_hip.so``.

The library is built in-tree by :func:`nvsubquadratic_amd.build.build_library`
(called from ``__graft_entry__.build()``).  Loading happens lazily on first use
so that importing the package never needs a GPU or a built library, mirroring
how the reference defers its native import until an op is called
(``nvsubquadratic/ops/fftconv_custom.py:96-109``).  A missing library or a
non-gfx950 device raises at call time with a clear message; there is no CPU
fallback on the product path.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch


__all__ = [
    "LIB_PATH",
    "NSQ_DTYPE",
    "HipLibraryError",
    "check",
    "dtype_code",
    "get_lib",
    "library_exports",
    "ptr",
    "stream_ptr",
]

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libnsq_hip.so")

NSQ_OK = 0
NSQ_DTYPE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}
NSQ_DIR_FWD = 0
NSQ_DIR_BWD = 1
ABI_VERSION = 16
NSQ_NOALLOC_SCRATCH_BYTES = 32 << 20  # include/nsq_hip.h: the fixed scratch of nsq_causal_conv1d_bwd_noalloc


class HipLibraryError(RuntimeError):
    """Raised when the native library is missing, incompatible or returns an error."""


_c_void_p = ctypes.c_void_p
_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_uint = ctypes.c_uint
_c_size = ctypes.c_size_t

# name -> (restype, argtypes).  Must match include/nsq_hip.h.
_SIGNATURES = {
    "nsq_abi_version": (_c_int, []),
    "nsq_last_error": (ctypes.c_char_p, []),
    "nsq_init": (_c_int, []),
    "nsq_fftconv1d_causal_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64, _c_int]),
    "nsq_fftconv1d_causal_fwd": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_void_p, _c_size, _c_void_p],
    ),
    "nsq_fftconv1d_causal_bwd": (
        _c_int,
        [
            _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int,
            _c_i64, _c_i64, _c_i64, _c_i64, _c_void_p, _c_size, _c_int, _c_void_p,
        ],
    ),
    "nsq_fftconv1d_causal_film_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int]),
    "nsq_fftconv1d_causal_film_fwd": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_void_p,
         _c_size, _c_void_p],
    ),
    "nsq_fftconv1d_causal_film_bwd": (
        _c_int,
        [
            _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int,
            _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_void_p, _c_size, _c_int, _c_void_p,
        ],
    ),
    "nsq_gated_fftconv1d_causal_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int]),
    "nsq_gated_fftconv1d_causal_fwd": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int,
         _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_void_p, _c_size, _c_void_p],
    ),
    "nsq_gated_fftconv1d_causal_bwd": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
         _c_void_p, _c_void_p, _c_int, _c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_void_p,
         _c_size, _c_void_p],
    ),
    "nsq_gated_fftconv_nd_workspace_bytes": (
        _c_size, [_c_int, _c_i64, _c_i64, ctypes.POINTER(_c_i64), ctypes.POINTER(_c_i64), _c_i64, _c_uint, _c_int, _c_int]),
    "nsq_gated_fftconv_nd_fwd": (
        _c_int,
        [_c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int,
         _c_i64, _c_i64, ctypes.POINTER(_c_i64), ctypes.POINTER(_c_i64), _c_i64, _c_uint, _c_void_p, _c_size, _c_void_p],
    ),
    "nsq_gated_fftconv_nd_bwd": (
        _c_int,
        [_c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
         _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int, _c_i64, _c_i64, ctypes.POINTER(_c_i64), ctypes.POINTER(_c_i64), _c_i64, _c_uint,
         _c_void_p, _c_size, _c_void_p],
    ),
    "nsq_circular_fftconv1d_fwd": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_void_p],
    ),
    "nsq_circular_fftconv1d_bwd": (
        _c_int,
        [
            _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int,
            _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_void_p,
        ],
    ),
    "nsq_mixed_fftconv1d_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_uint, _c_int, _c_int]),
    "nsq_mixed_fftconv1d_fwd": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_uint,
         _c_void_p, _c_size, _c_void_p],
    ),
    "nsq_mixed_fftconv1d_bwd": (
        _c_int,
        [
            _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int,
            _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_uint, _c_void_p, _c_size, _c_void_p,
        ],
    ),
    "nsq_causal_conv1d_fwd": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_void_p],
    ),
    "nsq_causal_conv1d_bwd_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64, _c_int]),
    "nsq_causal_conv1d_bwd": (
        _c_int,
        [
            _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int,
            _c_i64, _c_i64, _c_i64, _c_i64, _c_void_p, _c_size, _c_void_p,
        ],
    ),
    "nsq_causal_conv1d_bwd_noalloc": (
        _c_int,
        [
            _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int,
            _c_i64, _c_i64, _c_i64, _c_i64, _c_void_p,
        ],
    ),
    "nsq_siren_mlp_fwd": (
        _c_int,
        [_c_void_p, _c_i64, _c_int, _c_void_p, _c_void_p, _c_int, _c_void_p, _c_void_p, _c_int, _c_int, _c_void_p,
         _c_i64, _c_void_p],
    ),
    "nsq_siren_readout_fwd": (
        _c_int, [_c_void_p, _c_void_p, _c_i64, _c_int, _c_void_p, _c_i64, _c_i64, _c_void_p, _c_void_p]),
    "nsq_batched_transpose": (_c_int, [_c_void_p, _c_void_p, _c_int, _c_i64, _c_i64, _c_i64, _c_void_p]),
    "nsq_channel_rmsnorm_fwd": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_i64, _c_i64, _c_i64, ctypes.c_float, _c_int, _c_int,
         _c_void_p],
    ),
    "nsq_channel_l2norm_fwd": (
        _c_int, [_c_void_p, _c_void_p, _c_int, _c_i64, _c_i64, _c_i64, ctypes.c_float, _c_int, _c_void_p]),
    "nsq_channel_l2norm_bwd": (
        _c_int, [_c_void_p, _c_void_p, _c_void_p, _c_int, _c_i64, _c_i64, _c_i64, ctypes.c_float, _c_int, _c_void_p]),
    "nsq_channel_rmsnorm_bwd_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64]),
    "nsq_channel_layernorm_fwd": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_i64, _c_i64, _c_i64, ctypes.c_float, _c_int,
         _c_int, _c_void_p],
    ),
    "nsq_channel_layernorm_bwd_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64]),
    "nsq_channel_layernorm_bwd": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_i64,
         _c_i64, _c_i64, ctypes.c_float, _c_int, _c_int, _c_void_p, _c_size, _c_void_p],
    ),
    "nsq_channel_groupnorm_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64, _c_int]),
    "nsq_channel_groupnorm_fwd": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_i64, _c_i64, _c_i64,
         _c_i64, ctypes.c_float, _c_int, _c_void_p, _c_size, _c_void_p],
    ),
    "nsq_channel_groupnorm_bwd": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
         _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_void_p, _c_size, _c_void_p],
    ),
    "nsq_channel_rmsnorm_bwd": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_i64, _c_i64, _c_i64,
         ctypes.c_float, _c_int, _c_int, _c_void_p, _c_size, _c_void_p],
    ),
    "nsq_siren_readout_bwd_workspace_bytes": (_c_size, [_c_i64, _c_int, _c_i64, _c_i64]),
    "nsq_siren_fftconv1d_causal_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64, _c_int]),
    "nsq_siren_fftconv1d_causal_fwd": (
        _c_int, [_c_void_p, _c_void_p, _c_i64, _c_void_p, _c_void_p, _c_int, _c_void_p, _c_void_p, _c_int, _c_i64,
                 _c_i64, _c_i64, _c_i64, _c_void_p, _c_size, _c_void_p]),
    "nsq_siren_fftconv1d_causal_bwd": (
        _c_int, [_c_void_p, _c_void_p, _c_void_p, _c_i64, _c_void_p, _c_void_p, _c_int, _c_void_p, _c_void_p,
                 _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_void_p,
                 _c_size, _c_int, _c_void_p]),
    "nsq_siren_readout_bwd": (
        _c_int, [_c_void_p, _c_i64, _c_void_p, _c_i64, _c_void_p, _c_i64, _c_int, _c_i64, _c_i64, _c_void_p,
                 _c_void_p, _c_void_p, _c_void_p, _c_size, _c_void_p]),
    "nsq_siren_mlp_film_fwd": (
        _c_int,
        [_c_void_p, _c_i64, _c_int, _c_void_p, _c_void_p, _c_int, _c_void_p, _c_void_p, _c_int, _c_int, _c_void_p,
         _c_i64, _c_int, _c_void_p, _c_i64, _c_void_p],
    ),
    "nsq_siren_film_readout_fwd": (
        _c_int, [_c_void_p, _c_void_p, _c_i64, _c_int, _c_void_p, _c_i64, _c_i64, _c_i64, _c_void_p, _c_void_p]),
    "nsq_siren_mlp_film_bwd_workspace_bytes": (_c_size, [_c_i64, _c_int, _c_int, _c_int, _c_int, _c_i64, _c_int]),
    "nsq_siren_mlp_film_bwd": (
        _c_int,
        [_c_void_p, _c_i64, _c_i64, _c_i64, _c_void_p, _c_i64, _c_int, _c_void_p, _c_void_p, _c_int, _c_void_p,
         _c_void_p, _c_int, _c_int, _c_void_p, _c_i64, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
         _c_void_p, _c_size, _c_void_p],
    ),
    "nsq_siren_mlp_bwd_workspace_bytes": (_c_size, [_c_i64, _c_int, _c_int, _c_int, _c_int]),
    "nsq_siren_mlp_bwd": (
        _c_int,
        [_c_void_p, _c_i64, _c_i64, _c_void_p, _c_i64, _c_int, _c_void_p, _c_void_p, _c_int, _c_void_p, _c_void_p,
         _c_int, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_size, _c_void_p],
    ),
    "nsq_b2b_causal_conv1d_fwd": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
         _c_void_p],
    ),
    "nsq_b2b_causal_conv1d_bwd_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64]),
    "nsq_b2b_causal_conv1d_bwd": (
        _c_int,
        [
            _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
            _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_void_p, _c_size, _c_void_p,
        ],
    ),
    "nsq_fftconv_nd_workspace_bytes": (
        _c_size, [_c_int, _c_i64, _c_i64, ctypes.POINTER(_c_i64), ctypes.POINTER(_c_i64), _c_i64, _c_int]),
    "nsq_fftconv_nd_fwd": (
        _c_int,
        [_c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_i64, _c_i64, ctypes.POINTER(_c_i64),
         ctypes.POINTER(_c_i64), _c_i64, _c_void_p, _c_size, _c_void_p],
    ),
    "nsq_fftconv_nd_bwd": (
        _c_int,
        [_c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_i64, _c_i64,
         ctypes.POINTER(_c_i64), ctypes.POINTER(_c_i64), _c_i64, _c_void_p, _c_size, _c_int, _c_void_p],
    ),
    "nsq_mixed_fftconv_nd_workspace_bytes": (
        _c_size, [_c_int, _c_i64, _c_i64, ctypes.POINTER(_c_i64), ctypes.POINTER(_c_i64), _c_i64, _c_uint, _c_int]),
    "nsq_mixed_fftconv_nd_fwd": (
        _c_int,
        [_c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_i64, _c_i64, ctypes.POINTER(_c_i64),
         ctypes.POINTER(_c_i64), _c_i64, _c_uint, _c_void_p, _c_size, _c_void_p],
    ),
    "nsq_mixed_fftconv_nd_bwd": (
        _c_int,
        [_c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_i64, _c_i64,
         ctypes.POINTER(_c_i64), ctypes.POINTER(_c_i64), _c_i64, _c_uint, _c_void_p, _c_size, _c_int, _c_void_p],
    ),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None
_checked_devices: set[int] = set()


def library_exports() -> list[str]:
    """Names of every C-ABI entry point the Python layer binds."""
    return sorted(_SIGNATURES)


def _load() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise HipLibraryError(
            f"nvsubquadratic_amd native library not found at {LIB_PATH}. "
            "Build it with `python -c 'import __graft_entry__ as g; g.build()'` "
            "(hipcc --offload-arch=gfx950)."
        )
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    ver = lib.nsq_abi_version()
    if ver != ABI_VERSION:
        raise HipLibraryError(f"libnsq_hip.so ABI version {ver} != expected {ABI_VERSION}; rebuild the library.")
    return lib


def get_lib() -> ctypes.CDLL:
    """Load (once) and return the native library."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                _lib = _load()
    return _lib


def check_device(t: torch.Tensor) -> None:
    """Fail loudly unless ``t`` lives on a gfx950 GPU."""
    if t.device.type != "cuda":
        raise HipLibraryError(
            f"fft_backend='hip' needs tensors on a ROCm GPU (got device {t.device}); there is no CPU fallback."
        )
    idx = t.device.index if t.device.index is not None else torch.cuda.current_device()
    if idx in _checked_devices:
        return
    arch = getattr(torch.cuda.get_device_properties(idx), "gcnArchName", "")
    if not arch.startswith("gfx950"):
        raise HipLibraryError(f"libnsq_hip.so is built for gfx950 only; device {idx} is {arch!r}.")
    _checked_devices.add(idx)


def check(rc: int) -> None:
    """Raise :class:`HipLibraryError` with the library's message when ``rc != 0``."""
    if rc != NSQ_OK:
        msg = get_lib().nsq_last_error().decode(errors="replace")
        if rc == 1:
            raise ValueError(msg)
        if rc == 2:
            raise NotImplementedError(msg)
        raise HipLibraryError(msg)


def dtype_code(dt: torch.dtype) -> int:
    try:
        return NSQ_DTYPE[dt]
    except KeyError as exc:
        raise TypeError(f"unsupported dtype {dt}; expected float32, bfloat16 or float16") from exc


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def i64_array(values) -> ctypes.Array:
    """Host int64 array argument (sizes of the N-d ops)."""
    vals = [int(v) for v in values]
    return (ctypes.c_int64 * len(vals))(*vals)


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream
