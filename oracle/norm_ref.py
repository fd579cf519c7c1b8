"""CPU oracle for the Hyena gate + channel RMSNorm + layout pass (test infrastructure only).

Restates, with torch on the CPU, the reference's op sequence at its norm sites:

- gate: ``y * gate_nonlinear(v)`` on I/O-dtype tensors (``nvsubquadratic/modules/hyena_nd.py:546`` and ``:570``);
- norm: ``_rmsnorm_pytorch`` (``nvsubquadratic/modules/rms_norm.py:71-77``): upcast to float32,
  ``x * rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)``, ``(weight * x).to(input_dtype)``, applied to
  ``u.movedim(1, -1)`` (``hyena_nd.py:573-580``); the channels-first module
  (``rms_norm_channel_first.py:71-80``) is the same along dim 1;
- layout: ``rearrange(y, "b c ... -> b ... c")`` (``hyena_nd.py:583``) for the channels-last output.

The backward is torch autograd through that sequence.  Pinned in ``tests/test_oracle_norm.py`` by a closed form of
the normalised values, scale invariance, finite-difference gradients (float64 gradcheck) and the orthogonality of
the input gradient to ``u`` at ``eps = 0``.

The QK-norm (``nvsubquadratic/utils/qk_norm.py``, ``L2Norm``: ``F.normalize(x, p=2, dim, eps)``) is restated as the
norm over ``dim`` accumulated in float32 and rounded to the input dtype (torch's vector norm of a 16-bit tensor),
clamped at ``eps``, and ``x / n`` in the input dtype; pinned against torch's own ``F.normalize`` (a library routine),
a closed form (3, 4) -> (0.6, 0.8), the clamp (a vector shorter than eps comes out as ``x / eps``) and float64
gradcheck.

The LayerNorm site (a ``torch.nn.LayerNorm(C)`` as ``pixelhyena_norm``, applied by ``hyena_nd.py:548-556`` to
``z.movedim(1, -1)``) is restated as torch's layer norm computes it: float32 arithmetic (the input upcast, the
parameters float32), the mean and the biased variance over the channels, ``(x - mean) * rsqrt(var + eps) * w + b``,
rounded once to the input dtype.  Pinned against ``torch.nn.functional.layer_norm`` in float64 (a library routine), a
closed form ((1, 2, 3) -> (-sqrt(3/2), 0, sqrt(3/2)) at eps = 0), shift and scale invariance of the normalised values,
and float64 gradcheck.

The GroupNorm site (a ``torch.nn.GroupNorm(num_groups, C)`` as ``pixelhyena_norm``, applied channels-first by
``hyena_nd.py:548-550`` since ``modules/_channels_first_utils.py:27`` marks GroupNorm channels-first) is restated as
torch's group norm computes it: per sample and group of ``C / G`` consecutive channels, the mean and the biased
variance over those channels and every position (accumulated in float64 here), then per channel the float32
scale ``a = rsqrt(var + eps) * w`` and shift ``h = b - mean * a``, ``x * a + h`` rounded once to the input dtype.
Pinned against ``torch.nn.functional.group_norm`` in float64 (a library routine), ``instance_norm`` at ``G = C`` (a
second library routine), a closed form at ``G = 1`` and float64 gradcheck.
"""

from __future__ import annotations

from typing import Optional

import torch

__all__ = ["gated_channel_groupnorm_ref", "gated_channel_layernorm_ref", "gated_channel_rmsnorm_ref", "l2norm_ref"]

_ACTS = {0: lambda t: t, 1: torch.sigmoid, 2: torch.nn.functional.silu}


def gated_channel_rmsnorm_ref(y: torch.Tensor, v: Optional[torch.Tensor], weight: torch.Tensor, eps: float,
                              act: int = 1, channels_last: bool = True) -> torch.Tensor:
    """``y``, ``v`` ``[B, C, *S]`` (any dtype, CPU), ``weight`` ``[C]`` -> ``[B, *S, C]`` or ``[B, C, *S]``."""
    u = y * _ACTS[act](v) if v is not None else y           # hyena_nd.py:570 (I/O dtype)
    x = u.movedim(1, -1)                                     # hyena_nd.py:578
    dt = x.dtype
    xf = x.to(torch.float32) if dt != torch.float64 else x   # rms_norm.py:73-74
    var = xf.pow(2).mean(-1, keepdim=True)                   # rms_norm.py:75
    xf = xf * torch.rsqrt(var + eps)                         # rms_norm.py:76
    out = (weight * xf).to(dt)                               # rms_norm.py:77
    return out if channels_last else out.movedim(-1, 1)


def l2norm_ref(x: torch.Tensor, dim: int = 1, eps: float = 1e-12) -> torch.Tensor:
    """``F.normalize(x, p=2, dim=dim, eps=eps)`` restated step by step (``qk_norm.py:109``)."""
    xf = x.to(torch.float32) if x.dtype != torch.float64 else x
    n = torch.linalg.vector_norm(xf, dim=dim, keepdim=True).to(x.dtype)  # torch's norm returns the input dtype
    n = n.clamp_min(eps)
    return (xf / n.to(xf.dtype)).to(x.dtype)


def gated_channel_layernorm_ref(y: torch.Tensor, v: Optional[torch.Tensor], weight: Optional[torch.Tensor],
                                bias: Optional[torch.Tensor], eps: float = 1e-5, act: int = 1,
                                channels_last: bool = False) -> torch.Tensor:
    """``y``, ``v`` ``[B, C, *S]`` (CPU), ``weight`` / ``bias`` ``[C]`` or None -> ``[B, *S, C]`` or ``[B, C, *S]``."""
    u = y * _ACTS[act](v) if v is not None else y           # hyena_nd.py:546 (I/O dtype)
    x = u.movedim(1, -1)                                     # hyena_nd.py:553-554 (rows of C channels)
    dt = x.dtype
    xf = x.to(torch.float32) if dt != torch.float64 else x
    mean = xf.mean(-1, keepdim=True)
    var = (xf - mean).pow(2).mean(-1, keepdim=True)          # biased, as LayerNorm
    out = (xf - mean) * torch.rsqrt(var + eps)
    if weight is not None:
        out = out * weight.to(xf.dtype)
    if bias is not None:
        out = out + bias.to(xf.dtype)
    out = out.to(dt)
    return out if channels_last else out.movedim(-1, 1)


def gated_channel_groupnorm_ref(y: torch.Tensor, v: Optional[torch.Tensor], weight: Optional[torch.Tensor],
                                bias: Optional[torch.Tensor], num_groups: int, eps: float = 1e-5,
                                act: int = 1) -> torch.Tensor:
    """``y``, ``v`` ``[B, C, *S]`` (CPU), ``weight`` / ``bias`` ``[C]`` or None -> ``[B, C, *S]``."""
    u = y * _ACTS[act](v) if v is not None else y           # hyena_nd.py:546 (I/O dtype)
    B, C = u.shape[:2]
    G = num_groups
    assert C % G == 0
    dt = u.dtype
    cdt = torch.float64 if dt == torch.float64 else torch.float32
    xg = u.reshape(B, G, -1).to(torch.float64)
    mean = xg.mean(-1)                                        # [B, G]
    var = (xg - mean[..., None]).pow(2).mean(-1)              # biased, as GroupNorm
    rstd = torch.rsqrt(var + eps).to(cdt)
    w = weight.to(cdt) if weight is not None else torch.ones(C, dtype=cdt)
    b = bias.to(cdt) if bias is not None else torch.zeros(C, dtype=cdt)
    a = rstd.repeat_interleave(C // G, dim=1) * w             # [B, C]
    h = b - mean.to(cdt).repeat_interleave(C // G, dim=1) * a
    x = u.reshape(B, C, -1).to(cdt)
    out = x * a[..., None] + h[..., None]
    return out.to(dt).reshape(u.shape)
