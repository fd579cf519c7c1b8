r"""Hyena's gate + RMSNorm over channels + layout change as one HIP pass.

The reference's Hyena operator normalises over channels at three sites, each a chain of elementwise ops and
layout copies around the long convolution (``nvsubquadratic/modules/hyena_nd.py``):

- ``:570-583``, the output: ``y = y * gate_nonlinear_2(value)``, then ``output_norm`` on
  ``y.movedim(1, -1)`` (an ``RMSNorm`` over the last axis, ``modules/rms_norm.py:71-77``), then
  ``rearrange(y, "b c ... -> b ... c")``;
- ``:546-556``, the conv's input: ``z = query * gate_nonlinear(key)``, then ``pixelhyena_norm`` over channels,
  handed to the conv channels-first;
- a channels-first norm module (``modules/rms_norm_channel_first.py:71-80``, ``RMSNormChannelFirst``) is the same
  arithmetic along dim 1.

:func:`gated_channel_rmsnorm` computes ``round(w * (u * rsqrt(mean_c u^2 + eps)))`` with
``u = round(y * round(act(v)))`` (or ``u = y``) in one read of ``y`` / ``v`` and one write of the output, in either
layout (``nsq_channel_rmsnorm_fwd``); its backward recomputes ``u`` and the per-position scale and writes
``dy``, ``dv`` and the weight gradient in one more pass (``nsq_channel_rmsnorm_bwd``).
"""

from __future__ import annotations

from typing import Optional

import torch
from torch.library import custom_op

from . import _lib
from .gated_fftconv_hip import gate_code
from .layout import channels_first_contiguous

__all__ = ["HipGroupNorm", "HipL2Norm", "HipLayerNormChannels", "HipRMSNormChannelFirst", "channel_l2norm",
           "channel_rmsnorm", "gated_channel_groupnorm", "gated_channel_layernorm", "gated_channel_rmsnorm",
           "hyena_output_norm"]


def _flat(t: torch.Tensor) -> torch.Tensor:
    """``[B, C, *S]`` -> contiguous ``[B, C, prod(S)]``."""
    return t.contiguous().reshape(t.shape[0], t.shape[1], -1)


@custom_op("nsq_hip::gated_channel_rmsnorm", mutates_args=())
def gated_channel_rmsnorm_op(y: torch.Tensor, v: Optional[torch.Tensor], weight: torch.Tensor, eps: float, act: int,
                             channels_last: bool) -> torch.Tensor:
    """y, v ``[B, C, S]`` contiguous, weight fp32 ``[C]`` -> ``[B, S, C]`` (channels_last) or ``[B, C, S]``."""
    lib = _lib.get_lib()
    _lib.check_device(y)
    B, C, S = y.shape
    out = torch.empty((B, S, C) if channels_last else (B, C, S), dtype=y.dtype, device=y.device)
    _lib.check(lib.nsq_channel_rmsnorm_fwd(y.data_ptr(), v.data_ptr() if v is not None else None, weight.data_ptr(),
                                           out.data_ptr(), _lib.dtype_code(y.dtype), B, C, S, float(eps), act,
                                           int(channels_last), _lib.stream_ptr(y.device)))
    return out


@gated_channel_rmsnorm_op.register_fake
def _(y, v, weight, eps, act, channels_last):
    B, C, S = y.shape
    return y.new_empty((B, S, C) if channels_last else (B, C, S))


@custom_op("nsq_hip::gated_channel_rmsnorm_backward", mutates_args=())
def gated_channel_rmsnorm_backward_op(dout: torch.Tensor, y: torch.Tensor, v: Optional[torch.Tensor],
                                      weight: torch.Tensor, eps: float, act: int,
                                      channels_last: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Returns ``(dy, dv, dw)``; ``dv`` is empty when ``v`` is None, ``dw`` fp32 ``[C]``."""
    lib = _lib.get_lib()
    _lib.check_device(y)
    B, C, S = y.shape
    dy = torch.empty_like(y)
    dv = torch.empty_like(v) if v is not None else y.new_empty(0)
    dw = torch.empty(C, dtype=torch.float32, device=y.device)
    ws = torch.empty(int(lib.nsq_channel_rmsnorm_bwd_workspace_bytes(B, C, S)), dtype=torch.uint8, device=y.device)
    _lib.check(lib.nsq_channel_rmsnorm_bwd(
        dout.data_ptr(), y.data_ptr(), v.data_ptr() if v is not None else None, weight.data_ptr(), dy.data_ptr(),
        dv.data_ptr() if v is not None else None, dw.data_ptr(), _lib.dtype_code(y.dtype), B, C, S, float(eps), act,
        int(channels_last), ws.data_ptr(), ws.numel(), _lib.stream_ptr(y.device)))
    return dy, dv, dw


@gated_channel_rmsnorm_backward_op.register_fake
def _(dout, y, v, weight, eps, act, channels_last):
    return torch.empty_like(y), (torch.empty_like(v) if v is not None else y.new_empty(0)), \
        y.new_empty(y.shape[1], dtype=torch.float32)


def _setup(ctx, inputs, output):
    y, v, weight, eps, act, channels_last = inputs
    ctx.save_for_backward(y, v, weight)
    ctx.cfg = (eps, act, channels_last)


def _backward(ctx, gout):
    y, v, weight = ctx.saved_tensors
    eps, act, channels_last = ctx.cfg
    dy, dv, dw = gated_channel_rmsnorm_backward_op(gout.contiguous(), y, v, weight, eps, act, channels_last)
    return dy, (dv if v is not None else None), dw, None, None, None


gated_channel_rmsnorm_op.register_autograd(_backward, setup_context=_setup)


class _WeightToF32(torch.autograd.Function):
    """The norm's weight as fp32 (the reference multiplies an fp32 tensor by it, so a 16-bit weight is promoted
    exactly); its gradient goes back in the weight's dtype."""

    @staticmethod
    def forward(ctx, w):
        ctx.dt = w.dtype
        return w.float()

    @staticmethod
    def backward(ctx, g):
        return g.to(ctx.dt)


def gated_channel_rmsnorm(y: torch.Tensor, v: Optional[torch.Tensor], weight: torch.Tensor, eps: float = 1e-6,
                          gate_nonlinear="sigmoid", channels_last_out: bool = True) -> torch.Tensor:
    """RMSNorm over channels of ``y * act(v)`` (of ``y`` when ``v`` is None), in one pass.

    Args:
        y, v: ``[B, C, *spatial]`` in fp32 / bf16 / fp16 (same dtype and shape).
        weight: ``[C]``, the norm's learned scale.
        eps: added to the mean square, as ``RMSNorm(eps=...)``.
        gate_nonlinear: ``"identity" | "sigmoid" | "silu"`` or the matching ``nn`` module.
        channels_last_out: ``True`` returns ``[B, *spatial, C]`` (the norm over ``movedim(1, -1)`` followed by the
            output rearrange), ``False`` returns ``[B, C, *spatial]``.
    """
    if y.dim() < 2:
        raise ValueError(f"expected [B, C, *spatial], got shape {tuple(y.shape)}")
    if v is not None and (v.shape != y.shape or v.dtype != y.dtype):
        raise ValueError(f"v {tuple(v.shape)} {v.dtype} must match y {tuple(y.shape)} {y.dtype}")
    if weight.shape != (y.shape[1],):
        raise ValueError(f"weight shape {tuple(weight.shape)} != ({y.shape[1]},)")
    shape = y.shape
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (y, v, weight)):
        # the backward's two LDS tiles take fewer channels than the forward's one (C <= 3536 against 7781): refuse
        # before the forward runs rather than at loss.backward()
        C, S = shape[1], max(1, y.numel() // max(1, shape[0] * shape[1]))
        if _lib.get_lib().nsq_channel_rmsnorm_bwd_workspace_bytes(shape[0], C, S) == 0:
            raise NotImplementedError(f"fft_backend='hip' channel RMSNorm backward: C={C} exceeds the backward's "
                                      f"LDS tiles (C <= 3536); the forward alone takes C <= 7781")
    w = _WeightToF32.apply(weight) if weight.dtype != torch.float32 else weight
    out = gated_channel_rmsnorm_op(_flat(y), _flat(v) if v is not None else None, w.contiguous(), float(eps),
                                   gate_code(gate_nonlinear) if v is not None else 0, bool(channels_last_out))
    if channels_last_out:
        return out.view(shape[0], *shape[2:], shape[1])
    return out.view(shape)


def channel_rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """``RMSNormChannelFirst`` arithmetic (``modules/rms_norm_channel_first.py:71-80``): ``x`` ``[B, C, *S]``."""
    return gated_channel_rmsnorm(x, None, weight, eps, "identity", channels_last_out=False)


def hyena_output_norm(y: torch.Tensor, value: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6,
                      gate_nonlinear_2="sigmoid") -> torch.Tensor:
    """The Hyena operator's tail (``hyena_nd.py:570-583``) with an RMSNorm ``output_norm``: ``y`` (the long
    conv's output) and ``value`` ``[B, C, *spatial]`` -> ``[B, *spatial, C]``."""
    return gated_channel_rmsnorm(y, value, weight, eps, gate_nonlinear_2, channels_last_out=True)


class HipRMSNormChannelFirst(torch.nn.Module):
    """Drop-in for ``RMSNormChannelFirst`` (``modules/rms_norm_channel_first.py:83``): normalises ``[B, C, *S]``
    over dim 1 on the HIP kernel.  Same parameter (``weight``, ones) and ``eps``; the ``channels_first`` flag lets
    the Hyena operator skip its ``movedim`` round trip."""

    channels_first: bool = True

    def __init__(self, dim: int, eps: float = 1e-6):
        super().__init__()
        self.weight = torch.nn.Parameter(torch.ones(dim))
        self.weight._no_weight_decay = True
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return channel_rmsnorm(x, self.weight, self.eps)


# ---------------------------------------------------------------------------
# LayerNorm over channels at the pixelhyena_norm site (a torch.nn.LayerNorm(C) in the reference's configs, applied by
# modules/hyena_nd.py:548-556 to z moved channels-last), one HIP pass each way (nsq_channel_layernorm_fwd / _bwd)
# ---------------------------------------------------------------------------
@custom_op("nsq_hip::gated_channel_layernorm", mutates_args=())
def gated_channel_layernorm_op(y: torch.Tensor, v: Optional[torch.Tensor], weight: Optional[torch.Tensor],
                               bias: Optional[torch.Tensor], eps: float, act: int,
                               channels_last: bool) -> torch.Tensor:
    """y, v ``[B, C, S]`` contiguous, weight / bias fp32 ``[C]`` or None -> ``[B, S, C]`` or ``[B, C, S]``."""
    lib = _lib.get_lib()
    _lib.check_device(y)
    B, C, S = y.shape
    out = torch.empty((B, S, C) if channels_last else (B, C, S), dtype=y.dtype, device=y.device)
    _lib.check(lib.nsq_channel_layernorm_fwd(
        y.data_ptr(), v.data_ptr() if v is not None else None, weight.data_ptr() if weight is not None else None,
        bias.data_ptr() if bias is not None else None, out.data_ptr(), _lib.dtype_code(y.dtype), B, C, S, float(eps),
        act, int(channels_last), _lib.stream_ptr(y.device)))
    return out


@gated_channel_layernorm_op.register_fake
def _(y, v, weight, bias, eps, act, channels_last):
    B, C, S = y.shape
    return y.new_empty((B, S, C) if channels_last else (B, C, S))


@custom_op("nsq_hip::gated_channel_layernorm_backward", mutates_args=())
def gated_channel_layernorm_backward_op(dout: torch.Tensor, y: torch.Tensor, v: Optional[torch.Tensor],
                                        weight: Optional[torch.Tensor], want_db: bool, eps: float, act: int,
                                        channels_last: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor,
                                                                      torch.Tensor]:
    """Returns ``(dy, dv, dw, db)``; ``dv`` / ``dw`` / ``db`` are empty when ``v`` / ``weight`` / ``want_db`` are
    absent; ``dw`` and ``db`` fp32 ``[C]``."""
    lib = _lib.get_lib()
    _lib.check_device(y)
    B, C, S = y.shape
    dy = torch.empty_like(y)
    dv = torch.empty_like(v) if v is not None else y.new_empty(0)
    dw = torch.empty(C, dtype=torch.float32, device=y.device) if weight is not None else y.new_empty(0)
    db = torch.empty(C, dtype=torch.float32, device=y.device) if want_db else y.new_empty(0)
    nws = int(lib.nsq_channel_layernorm_bwd_workspace_bytes(B, C, S)) if (weight is not None or want_db) else 0
    ws = torch.empty(nws, dtype=torch.uint8, device=y.device)
    _lib.check(lib.nsq_channel_layernorm_bwd(
        dout.data_ptr(), y.data_ptr(), v.data_ptr() if v is not None else None,
        weight.data_ptr() if weight is not None else None, dy.data_ptr(), dv.data_ptr() if v is not None else None,
        dw.data_ptr() if weight is not None else None, db.data_ptr() if want_db else None, _lib.dtype_code(y.dtype),
        B, C, S, float(eps), act, int(channels_last), ws.data_ptr() if nws else None, nws,
        _lib.stream_ptr(y.device)))
    return dy, dv, dw, db


@gated_channel_layernorm_backward_op.register_fake
def _(dout, y, v, weight, want_db, eps, act, channels_last):
    C = y.shape[1]
    return (torch.empty_like(y), (torch.empty_like(v) if v is not None else y.new_empty(0)),
            (y.new_empty(C, dtype=torch.float32) if weight is not None else y.new_empty(0)),
            (y.new_empty(C, dtype=torch.float32) if want_db else y.new_empty(0)))


def _ln_setup(ctx, inputs, output):
    y, v, weight, bias, eps, act, channels_last = inputs
    ctx.save_for_backward(y, v, weight)
    ctx.cfg = (bias is not None, eps, act, channels_last)


def _ln_backward(ctx, gout):
    y, v, weight = ctx.saved_tensors
    has_b, eps, act, channels_last = ctx.cfg
    dy, dv, dw, db = gated_channel_layernorm_backward_op(gout.contiguous(), y, v, weight, has_b, eps, act,
                                                         channels_last)
    return (dy, (dv if v is not None else None), (dw if weight is not None else None), (db if has_b else None),
            None, None, None)


gated_channel_layernorm_op.register_autograd(_ln_backward, setup_context=_ln_setup)


def gated_channel_layernorm(y: torch.Tensor, v: Optional[torch.Tensor], weight: Optional[torch.Tensor],
                            bias: Optional[torch.Tensor], eps: float = 1e-5, gate_nonlinear="sigmoid",
                            channels_last_out: bool = False) -> torch.Tensor:
    """``torch.nn.LayerNorm(C)`` over the channels of ``y * act(v)`` (of ``y`` when ``v`` is None), in one pass.

    Args:
        y, v: ``[B, C, *spatial]`` in fp32 / bf16 / fp16 (same dtype and shape).
        weight, bias: ``[C]`` or None (``elementwise_affine=False`` / ``bias=False``).
        eps: added to the variance, as ``LayerNorm(eps=...)``.
        gate_nonlinear: ``"identity" | "sigmoid" | "silu"`` or the matching ``nn`` module.
        channels_last_out: ``True`` returns ``[B, *spatial, C]``, ``False`` ``[B, C, *spatial]``.
    """
    if y.dim() < 2:
        raise ValueError(f"expected [B, C, *spatial], got shape {tuple(y.shape)}")
    if v is not None and (v.shape != y.shape or v.dtype != y.dtype):
        raise ValueError(f"v {tuple(v.shape)} {v.dtype} must match y {tuple(y.shape)} {y.dtype}")
    for name, t in (("weight", weight), ("bias", bias)):
        if t is not None and t.shape != (y.shape[1],):
            raise ValueError(f"{name} shape {tuple(t.shape)} != ({y.shape[1]},)")
    shape = y.shape
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (y, v, weight, bias)):
        C, S = shape[1], max(1, y.numel() // max(1, shape[0] * shape[1]))
        if _lib.get_lib().nsq_channel_layernorm_bwd_workspace_bytes(shape[0], C, S) == 0:
            raise NotImplementedError(f"fft_backend='hip' channel LayerNorm backward: C={C} exceeds the backward's "
                                      f"LDS tiles (C <= 3241); the forward alone takes C <= 7781")
    w = _WeightToF32.apply(weight) if weight is not None and weight.dtype != torch.float32 else weight
    b = _WeightToF32.apply(bias) if bias is not None and bias.dtype != torch.float32 else bias
    out = gated_channel_layernorm_op(_flat(y), _flat(v) if v is not None else None,
                                     w.contiguous() if w is not None else None, b.contiguous() if b is not None else None,
                                     float(eps), gate_code(gate_nonlinear) if v is not None else 0,
                                     bool(channels_last_out))
    if channels_last_out:
        return out.view(shape[0], *shape[2:], shape[1])
    return out.view(shape)


class HipLayerNormChannels(torch.nn.Module):
    """Drop-in for ``torch.nn.LayerNorm(C)`` at the Hyena operator's norm sites: the same parameters (``weight``
    ones, ``bias`` zeros, ``eps`` 1e-5, ``elementwise_affine``, ``bias``) and arithmetic, normalising
    ``[B, C, *spatial]`` over dim 1 on the HIP kernel.  ``channels_first = True`` lets the operator hand it the
    channels-first tensor (``hyena_nd.py:548-552``) instead of its ``movedim`` / ``reshape`` round trip."""

    channels_first: bool = True

    def __init__(self, normalized_shape, eps: float = 1e-5, elementwise_affine: bool = True, bias: bool = True,
                 device=None, dtype=None):
        super().__init__()
        shape = (normalized_shape,) if isinstance(normalized_shape, int) else tuple(normalized_shape)
        if len(shape) != 1:
            raise NotImplementedError(f"fft_backend='hip' LayerNorm normalises the channel axis only; got "
                                      f"normalized_shape={shape}")
        self.normalized_shape = shape
        self.eps = eps
        self.elementwise_affine = elementwise_affine
        kw = {"device": device, "dtype": dtype}
        if elementwise_affine:
            self.weight = torch.nn.Parameter(torch.ones(shape, **kw))
            self.bias = torch.nn.Parameter(torch.zeros(shape, **kw)) if bias else None
        else:
            self.register_parameter("weight", None)
            self.register_parameter("bias", None)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return gated_channel_layernorm(x, None, self.weight, self.bias, self.eps, "identity", channels_last_out=False)

    def extra_repr(self) -> str:
        return f"{self.normalized_shape}, eps={self.eps}, elementwise_affine={self.elementwise_affine}"


# ---------------------------------------------------------------------------
# GroupNorm over channels, channels-first (the pixelhyena_norm site with torch.nn.GroupNorm(G, C), applied by
# modules/hyena_nd.py:548-550 to z as it is), three passes each way (nsq_channel_groupnorm_fwd / _bwd)
# ---------------------------------------------------------------------------
@custom_op("nsq_hip::gated_channel_groupnorm", mutates_args=())
def gated_channel_groupnorm_op(y: torch.Tensor, v: Optional[torch.Tensor], weight: Optional[torch.Tensor],
                               bias: Optional[torch.Tensor], num_groups: int, eps: float,
                               act: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """y, v ``[B, C, S]`` contiguous, weight / bias fp32 ``[C]`` or None -> ``(out [B, C, S], mean [B, G],
    rstd [B, G])``, the statistics fp32."""
    lib = _lib.get_lib()
    _lib.check_device(y)
    B, C, S = y.shape
    out = torch.empty_like(y)
    mean = torch.empty((B, num_groups), dtype=torch.float32, device=y.device)
    rstd = torch.empty((B, num_groups), dtype=torch.float32, device=y.device)
    nws = int(lib.nsq_channel_groupnorm_workspace_bytes(B, C, num_groups, _lib.NSQ_DIR_FWD))
    ws = torch.empty(nws, dtype=torch.uint8, device=y.device)
    _lib.check(lib.nsq_channel_groupnorm_fwd(
        y.data_ptr(), v.data_ptr() if v is not None else None, weight.data_ptr() if weight is not None else None,
        bias.data_ptr() if bias is not None else None, out.data_ptr(), mean.data_ptr(), rstd.data_ptr(),
        _lib.dtype_code(y.dtype), B, C, S, num_groups, float(eps), act, ws.data_ptr() if nws else None, nws,
        _lib.stream_ptr(y.device)))
    return out, mean, rstd


@gated_channel_groupnorm_op.register_fake
def _(y, v, weight, bias, num_groups, eps, act):
    B = y.shape[0]
    return (torch.empty_like(y), y.new_empty((B, num_groups), dtype=torch.float32),
            y.new_empty((B, num_groups), dtype=torch.float32))


@custom_op("nsq_hip::gated_channel_groupnorm_backward", mutates_args=())
def gated_channel_groupnorm_backward_op(dout: torch.Tensor, y: torch.Tensor, v: Optional[torch.Tensor],
                                        weight: Optional[torch.Tensor], mean: torch.Tensor, rstd: torch.Tensor,
                                        want_db: bool, act: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor,
                                                                          torch.Tensor]:
    """Returns ``(dy, dv, dw, db)``; ``dv`` / ``dw`` / ``db`` are empty when ``v`` / ``weight`` / ``want_db`` are
    absent; ``dw`` and ``db`` fp32 ``[C]``."""
    lib = _lib.get_lib()
    _lib.check_device(y)
    B, C, S = y.shape
    G = mean.shape[1]
    dy = torch.empty_like(y)
    dv = torch.empty_like(v) if v is not None else y.new_empty(0)
    dw = torch.empty(C, dtype=torch.float32, device=y.device) if weight is not None else y.new_empty(0)
    db = torch.empty(C, dtype=torch.float32, device=y.device) if want_db else y.new_empty(0)
    nws = int(lib.nsq_channel_groupnorm_workspace_bytes(B, C, G, _lib.NSQ_DIR_BWD))
    ws = torch.empty(nws, dtype=torch.uint8, device=y.device)
    _lib.check(lib.nsq_channel_groupnorm_bwd(
        dout.data_ptr(), y.data_ptr(), v.data_ptr() if v is not None else None,
        weight.data_ptr() if weight is not None else None, mean.data_ptr(), rstd.data_ptr(), dy.data_ptr(),
        dv.data_ptr() if v is not None else None, dw.data_ptr() if weight is not None else None,
        db.data_ptr() if want_db else None, _lib.dtype_code(y.dtype), B, C, S, G, act, ws.data_ptr(), nws,
        _lib.stream_ptr(y.device)))
    return dy, dv, dw, db


@gated_channel_groupnorm_backward_op.register_fake
def _(dout, y, v, weight, mean, rstd, want_db, act):
    C = y.shape[1]
    return (torch.empty_like(y), (torch.empty_like(v) if v is not None else y.new_empty(0)),
            (y.new_empty(C, dtype=torch.float32) if weight is not None else y.new_empty(0)),
            (y.new_empty(C, dtype=torch.float32) if want_db else y.new_empty(0)))


def _gn_setup(ctx, inputs, output):
    y, v, weight, bias, num_groups, eps, act = inputs
    _, mean, rstd = output
    ctx.save_for_backward(y, v, weight, mean, rstd)
    ctx.cfg = (bias is not None, act)


def _gn_backward(ctx, gout, gmean, grstd):
    y, v, weight, mean, rstd = ctx.saved_tensors
    has_b, act = ctx.cfg
    dy, dv, dw, db = gated_channel_groupnorm_backward_op(gout.contiguous(), y, v, weight, mean, rstd, has_b, act)
    return (dy, (dv if v is not None else None), (dw if weight is not None else None), (db if has_b else None),
            None, None, None)


gated_channel_groupnorm_op.register_autograd(_gn_backward, setup_context=_gn_setup)


def gated_channel_groupnorm(y: torch.Tensor, v: Optional[torch.Tensor], weight: Optional[torch.Tensor],
                            bias: Optional[torch.Tensor], num_groups: int, eps: float = 1e-5,
                            gate_nonlinear="sigmoid") -> torch.Tensor:
    """``torch.nn.GroupNorm(num_groups, C)`` of ``y * act(v)`` (of ``y`` when ``v`` is None), channels-first.

    Args:
        y, v: ``[B, C, *spatial]`` in fp32 / bf16 / fp16 (same dtype and shape).
        weight, bias: ``[C]`` or None (``affine=False``).
        num_groups: groups of ``C / num_groups`` consecutive channels; ``C`` must be a multiple of it.
        eps: added to the variance, as ``GroupNorm(eps=...)``.
        gate_nonlinear: ``"identity" | "sigmoid" | "silu"`` or the matching ``nn`` module.
    """
    if y.dim() < 2:
        raise ValueError(f"expected [B, C, *spatial], got shape {tuple(y.shape)}")
    if v is not None and (v.shape != y.shape or v.dtype != y.dtype):
        raise ValueError(f"v {tuple(v.shape)} {v.dtype} must match y {tuple(y.shape)} {y.dtype}")
    C = y.shape[1]
    if num_groups < 1 or C % num_groups:
        raise ValueError(f"num_channels {C} must be divisible by num_groups {num_groups}")
    for name, t in (("weight", weight), ("bias", bias)):
        if t is not None and t.shape != (C,):
            raise ValueError(f"{name} shape {tuple(t.shape)} != ({C},)")
    w = _WeightToF32.apply(weight) if weight is not None and weight.dtype != torch.float32 else weight
    b = _WeightToF32.apply(bias) if bias is not None and bias.dtype != torch.float32 else bias
    out, _, _ = gated_channel_groupnorm_op(_flat(y), _flat(v) if v is not None else None,
                                           w.contiguous() if w is not None else None,
                                           b.contiguous() if b is not None else None, int(num_groups), float(eps),
                                           gate_code(gate_nonlinear) if v is not None else 0)
    return out.view(y.shape)


class HipGroupNorm(torch.nn.Module):
    """Drop-in for ``torch.nn.GroupNorm(num_groups, num_channels)`` at the Hyena operator's pixelhyena_norm site:
    the same parameters (``weight`` ones, ``bias`` zeros, ``eps`` 1e-5, ``affine``) and arithmetic over
    ``[B, C, *spatial]`` on the HIP kernels.  Channels-first like GroupNorm (``channels_first = True``)."""

    channels_first: bool = True

    def __init__(self, num_groups: int, num_channels: int, eps: float = 1e-5, affine: bool = True, device=None,
                 dtype=None):
        super().__init__()
        if num_channels % num_groups:
            raise ValueError("num_channels must be divisible by num_groups")
        self.num_groups = num_groups
        self.num_channels = num_channels
        self.eps = eps
        self.affine = affine
        kw = {"device": device, "dtype": dtype}
        if affine:
            self.weight = torch.nn.Parameter(torch.ones(num_channels, **kw))
            self.bias = torch.nn.Parameter(torch.zeros(num_channels, **kw))
        else:
            self.register_parameter("weight", None)
            self.register_parameter("bias", None)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return gated_channel_groupnorm(x, None, self.weight, self.bias, self.num_groups, self.eps, "identity")

    def extra_repr(self) -> str:
        return f"{self.num_groups}, {self.num_channels}, eps={self.eps}, affine={self.affine}"


# ---------------------------------------------------------------------------
# QK-norm: L2 normalisation over channels (nvsubquadratic/utils/qk_norm.py L2Norm, the q / k norm of
# modules/hyena_nd.py:529-543), one HIP pass each way (nsq_channel_l2norm_fwd / _bwd)
# ---------------------------------------------------------------------------
@custom_op("nsq_hip::channel_l2norm", mutates_args=())
def channel_l2norm_op(x: torch.Tensor, eps: float, channels_last: bool) -> torch.Tensor:
    """x ``[B, C, S]`` contiguous -> ``x / max(||x||_C, eps)`` as ``[B, S, C]`` (channels_last) or ``[B, C, S]``."""
    lib = _lib.get_lib()
    _lib.check_device(x)
    B, C, S = x.shape
    out = torch.empty((B, S, C) if channels_last else (B, C, S), dtype=x.dtype, device=x.device)
    _lib.check(lib.nsq_channel_l2norm_fwd(x.data_ptr(), out.data_ptr(), _lib.dtype_code(x.dtype), B, C, S,
                                          float(eps), int(channels_last), _lib.stream_ptr(x.device)))
    return out


@channel_l2norm_op.register_fake
def _(x, eps, channels_last):
    B, C, S = x.shape
    return x.new_empty((B, S, C) if channels_last else (B, C, S))


@custom_op("nsq_hip::channel_l2norm_backward", mutates_args=())
def channel_l2norm_backward_op(dout: torch.Tensor, x: torch.Tensor, eps: float, channels_last: bool) -> torch.Tensor:
    """dx ``[B, C, S]`` for dout in the forward output's layout."""
    lib = _lib.get_lib()
    _lib.check_device(x)
    B, C, S = x.shape
    dx = torch.empty_like(x)
    _lib.check(lib.nsq_channel_l2norm_bwd(dout.data_ptr(), x.data_ptr(), dx.data_ptr(), _lib.dtype_code(x.dtype), B,
                                          C, S, float(eps), int(channels_last), _lib.stream_ptr(x.device)))
    return dx


@channel_l2norm_backward_op.register_fake
def _(dout, x, eps, channels_last):
    return torch.empty_like(x)


def _l2_setup(ctx, inputs, output):
    x, eps, channels_last = inputs
    ctx.save_for_backward(x)
    ctx.cfg = (eps, channels_last)


def _l2_backward(ctx, gout):
    (x,) = ctx.saved_tensors
    eps, channels_last = ctx.cfg
    return channel_l2norm_backward_op(gout.contiguous(), x, eps, channels_last), None, None


channel_l2norm_op.register_autograd(_l2_backward, setup_context=_l2_setup)


def channel_l2norm(x: torch.Tensor, eps: float = 1e-12, channels_last_out: bool = False) -> torch.Tensor:
    """``F.normalize(x, p=2, dim=1, eps)`` for ``x [B, C, *spatial]`` (fp32 / bf16 / fp16) in one pass; with
    ``channels_last_out`` the result comes back as ``[B, *spatial, C]`` (normalised over its last axis)."""
    if x.dim() < 2:
        raise ValueError(f"expected [B, C, *spatial], got shape {tuple(x.shape)}")
    shape = x.shape
    if torch.is_grad_enabled() and x.requires_grad:
        C, S = shape[1], max(1, x.numel() // max(1, shape[0] * shape[1]))
        if _lib.get_lib().nsq_channel_rmsnorm_bwd_workspace_bytes(shape[0], C, S) == 0:  # same LDS tiles
            raise NotImplementedError(f"fft_backend='hip' channel L2 norm backward: C={C} exceeds the backward's "
                                      f"LDS tiles (C <= 3536); the forward alone takes C <= 7781")
    out = channel_l2norm_op(_flat(x), float(eps), bool(channels_last_out))
    if channels_last_out:
        return out.view(shape[0], *shape[2:], shape[1])
    return out.view(shape)


class HipL2Norm(torch.nn.Module):
    """Drop-in for ``L2Norm`` (``nvsubquadratic/utils/qk_norm.py``): ``F.normalize(x, p=2, dim=self.dim, eps)``
    with no parameters, and the same ``channels_first`` duck type (``dim == 1``) the Hyena operator uses to pick the
    layout (``hyena_nd.py:529-543``).  ``dim = 1`` normalises ``[B, C, *spatial]`` in place of layout; ``dim = -1``
    normalises ``[..., C]``: a channels-first tensor viewed channels-last (the Hyena operator's ``movedim``) is read
    as it lies, a contiguous channels-last one is moved channels-first once (``nsq_batched_transpose``); either way
    the result comes back ``[..., C]`` from the kernel's channels-last store."""

    def __init__(self, dim: int = -1, eps: float = 1e-12):
        super().__init__()
        self.dim = dim
        self.eps = eps

    @property
    def channels_first(self) -> bool:
        return self.dim == 1

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        d = self.dim % x.dim()
        if d == 1 and x.dim() >= 2:
            return channel_l2norm(x, self.eps)
        if d == x.dim() - 1 and x.dim() >= 2:
            xc = channels_first_contiguous(x.movedim(-1, 1))
            return channel_l2norm(xc, self.eps, channels_last_out=True)
        raise NotImplementedError(f"fft_backend='hip' L2Norm: dim={self.dim} on a {x.dim()}-d tensor (the HIP kernel "
                                  f"normalises the channel axis: dim 1 or -1)")

    def extra_repr(self) -> str:
        return f"dim={self.dim}, eps={self.eps}"
