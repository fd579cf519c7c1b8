"""HIP (gfx950) direct causal convolutions with the reference's call signatures.

Counterpart of ``nvsubquadratic/ops/causal_conv1d_custom.py``:

* :func:`causal_conv1d` -- depthwise causal conv (``causal_conv1d_custom.py:81-98``),
  nn.Conv1d tap order with left padding ``K-1``, optional bias, activation
  ``"identity"`` or ``"silu"``, ``1 <= K <= 256``; differentiable in x, weight
  and bias.
* :func:`b2b_causal_conv1d` -- fused back-to-back block
  (``causal_conv1d_custom.py:101-121``): projection conv on all ``3C`` channels,
  pre-gate ``z = k * v``, mixer conv with skip ``h = conv(z) + skip * z``,
  post-gate ``y = q * h``; differentiable in all inputs.

Both compute in fp32 and return ``x.dtype``; weights are used in fp32 (their
gradients flow back through the cast).  There is no CPU path.
"""

from __future__ import annotations

from typing import Optional

import torch
from torch.library import custom_op

from . import _lib


__all__ = ["b2b_causal_conv1d", "causal_conv1d"]

_ACT = {"identity": 0, "silu": 1}


def _io(x: torch.Tensor) -> tuple[torch.Tensor, torch.dtype]:
    dt = x.dtype if x.dtype in _lib.NSQ_DTYPE else torch.float32
    return x.to(dt).contiguous(), dt


@custom_op("nsq_hip::causal_conv1d", mutates_args=())
def causal_conv1d_op(x: torch.Tensor, w: torch.Tensor, bias: Optional[torch.Tensor], act: int) -> torch.Tensor:
    """Depthwise causal conv forward: x ``[B, C, L]`` contiguous (f32/bf16/f16), w ``[C, K]`` and bias ``[C]`` float32."""
    lib = _lib.get_lib()
    _lib.check_device(x)
    B, C, L = x.shape
    y = torch.empty_like(x)
    _lib.check(lib.nsq_causal_conv1d_fwd(
        x.data_ptr(), w.data_ptr(), _lib.ptr(bias), y.data_ptr(), _lib.dtype_code(x.dtype), act, B, C, L,
        w.shape[-1], _lib.stream_ptr(x.device)))
    return y


@causal_conv1d_op.register_fake
def _(x, w, bias, act):
    return torch.empty_like(x)


@custom_op("nsq_hip::causal_conv1d_backward", mutates_args=())
def causal_conv1d_backward_op(g: torch.Tensor, x: torch.Tensor, w: torch.Tensor, bias: Optional[torch.Tensor],
                              act: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``(gx, gw, gbias)``; gbias is empty when there is no bias."""
    lib = _lib.get_lib()
    B, C, L = x.shape
    K = w.shape[-1]
    gx = torch.empty_like(x)
    gw = torch.empty_like(w)
    gb = torch.empty(C if bias is not None else 0, dtype=torch.float32, device=x.device)
    need = lib.nsq_causal_conv1d_bwd_workspace_bytes(B, C, L, K, act)
    ws = torch.empty(need, dtype=torch.uint8, device=x.device) if need else None
    _lib.check(lib.nsq_causal_conv1d_bwd(
        g.data_ptr(), x.data_ptr(), w.data_ptr(), _lib.ptr(bias), gx.data_ptr(), gw.data_ptr(),
        gb.data_ptr() if bias is not None else None, _lib.dtype_code(x.dtype), act, B, C, L, K, _lib.ptr(ws), need,
        _lib.stream_ptr(x.device)))
    return gx, gw, gb


@causal_conv1d_backward_op.register_fake
def _(g, x, w, bias, act):
    return torch.empty_like(x), torch.empty_like(w), x.new_empty(x.shape[1] if bias is not None else 0,
                                                                 dtype=torch.float32)


def _cc_setup(ctx, inputs, output):
    x, w, bias, act = inputs
    ctx.save_for_backward(x, w, bias)
    ctx.act = act


def _cc_backward(ctx, gy):
    x, w, bias = ctx.saved_tensors
    gx, gw, gb = causal_conv1d_backward_op(gy.to(x.dtype).contiguous(), x, w, bias, ctx.act)
    return gx, gw, (gb if bias is not None else None), None


causal_conv1d_op.register_autograd(_cc_backward, setup_context=_cc_setup)


def causal_conv1d(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None = None,
    activation: str = "identity",
) -> torch.Tensor:
    """Depthwise causal 1D conv on the HIP backend.

    Args:
        x: Input ``[B, C, L]``.
        weight: Depthwise weight ``[C, K]``, ``1 <= K <= 256``.
        bias: Optional per-channel bias ``[C]``.
        activation: ``"identity"`` (default) or ``"silu"``.

    Returns:
        ``[B, C, L]`` in ``x.dtype``.
    """
    if activation not in _ACT:
        raise ValueError(f"activation must be 'identity' or 'silu'. Got {activation!r}.")
    if x.ndim != 3 or weight.ndim != 2 or weight.shape[0] != x.shape[1]:
        raise ValueError(f"expected x [B, C, L] and weight [C, K]; got {tuple(x.shape)} and {tuple(weight.shape)}")
    xc, _ = _io(x)
    wc = weight.float().contiguous()
    bc = None if bias is None else bias.float().contiguous()
    y = causal_conv1d_op(xc, wc, bc, _ACT[activation])
    return y.to(x.dtype)


@custom_op("nsq_hip::b2b_causal_conv1d", mutates_args=())
def b2b_causal_conv1d_op(x: torch.Tensor, wp: torch.Tensor, wm: torch.Tensor,
                         skip: Optional[torch.Tensor]) -> torch.Tensor:
    """Fused B2B forward: x ``[B, 3C, L]`` contiguous, wp ``[3C, Kp]``, wm ``[C, Km]``, skip ``[C]`` float32 or None."""
    lib = _lib.get_lib()
    _lib.check_device(x)
    B, C3, L = x.shape
    C = C3 // 3
    y = torch.empty(B, C, L, dtype=x.dtype, device=x.device)
    _lib.check(lib.nsq_b2b_causal_conv1d_fwd(
        x.data_ptr(), wp.data_ptr(), wm.data_ptr(), _lib.ptr(skip), y.data_ptr(), _lib.dtype_code(x.dtype),
        B, C, L, wp.shape[-1], wm.shape[-1], _lib.stream_ptr(x.device)))
    return y


@b2b_causal_conv1d_op.register_fake
def _(x, wp, wm, skip):
    return x.new_empty(x.shape[0], x.shape[1] // 3, x.shape[2])


@custom_op("nsq_hip::b2b_causal_conv1d_backward", mutates_args=())
def b2b_causal_conv1d_backward_op(g: torch.Tensor, x: torch.Tensor, wp: torch.Tensor, wm: torch.Tensor,
                                  skip: Optional[torch.Tensor]) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor,
                                                                         torch.Tensor]:
    """``(gx, gwp, gwm, gskip)``; gskip is empty when there is no skip."""
    lib = _lib.get_lib()
    B, C3, L = x.shape
    C = C3 // 3
    gx = torch.empty_like(x)
    gwp = torch.empty_like(wp)
    gwm = torch.empty_like(wm)
    gskip = torch.empty(C if skip is not None else 0, dtype=torch.float32, device=x.device)
    need = lib.nsq_b2b_causal_conv1d_bwd_workspace_bytes(B, C, L, wp.shape[-1], wm.shape[-1])
    ws = torch.empty(need, dtype=torch.uint8, device=x.device)
    _lib.check(lib.nsq_b2b_causal_conv1d_bwd(
        g.data_ptr(), x.data_ptr(), wp.data_ptr(), wm.data_ptr(), _lib.ptr(skip), gx.data_ptr(), gwp.data_ptr(),
        gwm.data_ptr(), gskip.data_ptr() if skip is not None else None, _lib.dtype_code(x.dtype), B, C, L,
        wp.shape[-1], wm.shape[-1], ws.data_ptr(), need, _lib.stream_ptr(x.device)))
    return gx, gwp, gwm, gskip


@b2b_causal_conv1d_backward_op.register_fake
def _(g, x, wp, wm, skip):
    return (torch.empty_like(x), torch.empty_like(wp), torch.empty_like(wm),
            x.new_empty(x.shape[1] // 3 if skip is not None else 0, dtype=torch.float32))


def _b2b_setup(ctx, inputs, output):
    ctx.save_for_backward(*inputs)


def _b2b_backward(ctx, gy):
    x, wp, wm, skip = ctx.saved_tensors
    gx, gwp, gwm, gskip = b2b_causal_conv1d_backward_op(gy.to(x.dtype).contiguous(), x, wp, wm, skip)
    return gx, gwp, gwm, (gskip if skip is not None else None)


b2b_causal_conv1d_op.register_autograd(_b2b_backward, setup_context=_b2b_setup)


def b2b_causal_conv1d(
    x: torch.Tensor,
    weight_proj: torch.Tensor,
    weight_mixer: torch.Tensor,
    skip_bias: torch.Tensor,
) -> torch.Tensor:
    """Fused back-to-back causal conv block on the HIP backend.

    Args:
        x: Input ``[B, 3*C, L]`` (channel order q | k | v).
        weight_proj: Projection weight ``[3*C, Kp]`` (depthwise).
        weight_mixer: Mixer weight ``[C, Km]`` (depthwise).
        skip_bias: Skip scale ``[C]`` (``None`` means 0).

    Returns:
        ``[B, C, L]`` in ``x.dtype``: ``q * (conv(k*v; weight_mixer) + skip * k*v)``
        with ``q, k, v`` the three channel groups of ``conv(x; weight_proj)``.
    """
    if x.ndim != 3 or x.shape[1] % 3 != 0:
        raise ValueError(f"x must be [B, 3*C, L]; got {tuple(x.shape)}")
    C = x.shape[1] // 3
    if weight_proj.shape[0] != 3 * C or weight_proj.ndim != 2:
        raise ValueError(f"weight_proj must be [3*C, K] = [{3 * C}, K]; got {tuple(weight_proj.shape)}")
    if weight_mixer.shape[0] != C or weight_mixer.ndim != 2:
        raise ValueError(f"weight_mixer must be [C, K] = [{C}, K]; got {tuple(weight_mixer.shape)}")
    if skip_bias is not None and skip_bias.shape != (C,):
        raise ValueError(f"skip_bias must be [C] = [{C}]; got {tuple(skip_bias.shape)}")
    xc, _ = _io(x)
    y = b2b_causal_conv1d_op(
        xc,
        weight_proj.float().contiguous(),
        weight_mixer.float().contiguous(),
        None if skip_bias is None else skip_bias.float().contiguous(),
    )
    return y.to(x.dtype)
