"""ctypes binding of ``oracle/direct_conv.c`` -- TEST INFRASTRUCTURE ONLY.

Brute-force float64 direct convolutions (no FFT).  These are the independent
closed forms that pin :mod:`oracle.fftconv_ref` and generate the golden
fixtures; see each C function's comment for the reference file:line it
restates.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np


_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_dp = ctypes.POINTER(ctypes.c_double)
_i64 = ctypes.c_int64


def build() -> str:
    """Compile ``direct_conv.c`` with gcc (in-tree, git-ignored)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def _get():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        lib.oracle_causal_conv1d.argtypes = [_dp, _dp, _dp, _i64, _i64, _i64, _i64]
        lib.oracle_causal_conv1d_bwd.argtypes = [_dp, _dp, _dp, _dp, _dp, _i64, _i64, _i64, _i64]
        lib.oracle_direct_causal_conv1d.argtypes = [_dp, _dp, ctypes.c_void_p, _dp, _i64, _i64, _i64, _i64]
        lib.oracle_conv3d_same.argtypes = [_dp, _dp, _dp] + [_i64] * 8
        _lib = lib
    return _lib


def _c(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float64))


def _p(a: np.ndarray):
    return a.ctypes.data_as(_dp)


def causal_conv1d(x, k) -> np.ndarray:
    """Reference causal FFT-conv semantics by brute force; x [B,H,L], k [H,K] -> [B,H,L] float64."""
    x, k = _c(x), _c(k)
    B, H, L = x.shape
    K = k.shape[-1]
    y = np.empty((B, H, L), dtype=np.float64)
    _get().oracle_causal_conv1d(_p(x), _p(k), _p(y), B, H, L, K)
    return y


def causal_conv1d_bwd(g, x, k) -> tuple[np.ndarray, np.ndarray]:
    """Adjoint of :func:`causal_conv1d`: (gx [B,H,L], gk [H,K]) in float64."""
    g, x, k = _c(g), _c(x), _c(k)
    B, H, L = x.shape
    K = k.shape[-1]
    gx = np.empty_like(x)
    gk = np.empty((H, K), dtype=np.float64)
    _get().oracle_causal_conv1d_bwd(_p(g), _p(x), _p(k), _p(gx), _p(gk), B, H, L, K)
    return gx, gk


def direct_causal_conv1d(x, w, bias=None) -> np.ndarray:
    """nn.Conv1d-order depthwise causal conv; x [B,C,L], w [C,K], bias [C] or None."""
    x, w = _c(x), _c(w)
    B, C, L = x.shape
    K = w.shape[-1]
    y = np.empty_like(x)
    b = None if bias is None else _c(bias)
    _get().oracle_direct_causal_conv1d(_p(x), _p(w), None if b is None else b.ctypes.data, _p(y), B, C, L, K)
    return y


def conv_same_nd(x, k) -> np.ndarray:
    """Non-causal 'same' depthwise conv for 1/2/3 spatial dims; x [B,H,*N], k [H,*K]."""
    x, k = _c(x), _c(k)
    nd = x.ndim - 2
    assert nd in (1, 2, 3) and k.ndim == nd + 1
    B, H = x.shape[:2]
    sp = list(x.shape[2:]) + [1] * (3 - nd)
    ks = list(k.shape[1:]) + [1] * (3 - nd)
    y = np.empty_like(x)
    _get().oracle_conv3d_same(_p(x), _p(k), _p(y), B, H, *sp, *ks)
    return y
