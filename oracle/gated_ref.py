"""Hyena-gated causal FFT conv restated on the CPU -- TEST INFRASTRUCTURE ONLY.

The composition of nvsubquadratic/modules/hyena_nd.py:546 (``query * gate(key)``),
:558 (CKConvND's global conv, ckconv_nd.py:1054-1062: the causal FFT conv of
fftconv.py:546-600 with its shortcut, restated by oracle.fftconv_ref) and :570
(``y * gate_2(value)``), with torch's own elementwise ops on the I/O dtype.
"""

from __future__ import annotations

import torch

from oracle.circular_ref import mixed_fftconv_torch
from oracle.fftconv_ref import causal_fftconv1d_torch

_GATES = {"identity": lambda t: t, "sigmoid": torch.sigmoid, "silu": torch.nn.functional.silu}


def gated_causal_fftconv1d_torch(q, k, v, kernel, shortcut=None, gate="silu", gate_2=None):
    g1 = _GATES[gate]
    g2 = _GATES[gate if gate_2 is None else gate_2]
    z = q * g1(k)
    y1 = causal_fftconv1d_torch(z, kernel, shortcut)
    return y1 * g2(v)


def gated_fftconv_nd_torch(q, k, v, kernel, periodic, shortcut=None, gate="silu", gate_2=None,
                           compute_dtype=torch.float32):
    """The same composition around the non-causal N-d conv of CKConvND (``ckconv_nd.py:1054-1062``: the
    zero-padded / circular / mixed op per axis, restated by ``oracle.circular_ref.mixed_fftconv_torch``)."""
    g1 = _GATES[gate]
    g2 = _GATES[gate if gate_2 is None else gate_2]
    z = q * g1(k)
    y1 = mixed_fftconv_torch(z, kernel, periodic, shortcut, compute_dtype=compute_dtype)
    return y1 * g2(v)
