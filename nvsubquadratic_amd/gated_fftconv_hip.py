r"""Hyena-gated FFT convolution (causal 1D, 2D / 3D) on the HIP backend.

The reference computes a Hyena layer's gated long convolution as separate ops
(``nvsubquadratic/modules/hyena_nd.py:546`` first gate, ``:558`` the CKConvND
global conv with its shortcut, ``ckconv_nd.py:1054-1062``, ``:570`` second gate):

    z  = query * gate_nonlinear(key)
    y1 = causal_fftconv1d(z, kernel) + shortcut * z
    y  = y1 * gate_nonlinear_2(value)

Each is an HBM round trip of a ``[B, H, L]`` tensor.  Here the forward's gates
run inside the conv's first-pass loader and last-pass epilogue (FFT lengths up
to 16384: one kernel), or as elementwise HIP kernels around the multi-kernel
conv (longer sequences).  The backward runs elementwise gate kernels around the
plain conv adjoint (a one-kernel gated adjoint measured slower on MI355X: a
latency-bound kernel at one workgroup per CU gains five operand streams).  2D / 3D: both directions
run the gates inside the N-d conv's first and last passes (z, or dy1 and dv, as
the first pass loads; gate 2, or dq and dk, in the last pass's epilogue) where
the plan has packed 2D rows with the vector epilogue or 3D plane passes, else as
gate kernels around the conv; both give the same bits.  Gates: ``"identity"``, ``"sigmoid"``, ``"silu"`` or the
matching ``torch.nn`` modules; ``gate_nonlinear_2=None`` reuses the first gate,
as ``Hyena.__init__`` does (``hyena_nd.py:274-278``).  Results follow the
reference composition with each elementwise product rounded to the I/O dtype.
"""

from __future__ import annotations

from typing import Optional

import torch
from torch.library import custom_op

from . import _lib
from .layout import channels_first_contiguous
from .fftconv_hip import _kernel_3d, _workspace
from .circular_fftconv_hip import needs_extension, periodic_by_extension
from .mixed_fftconv_hip import periodic_mask


__all__ = ["GATE_CODES", "gate_code", "hyena_gated_causal_fftconv1d_bhl", "gated_causal_fftconv1d_fwd_raw",
           "gated_causal_fftconv1d_bwd_raw", "hyena_gated_fftconv2d_bhl", "hyena_gated_fftconv3d_bhl",
           "hyena_gated_fftconv_nd_bhl"]

GATE_CODES = {"identity": 0, "sigmoid": 1, "silu": 2}
_MODULE_CODES = {torch.nn.Identity: 0, torch.nn.Sigmoid: 1, torch.nn.SiLU: 2}
_TORCH_GATES = {0: lambda t: t, 1: torch.sigmoid, 2: torch.nn.functional.silu}


def _aligned16(t: torch.Tensor) -> torch.Tensor:
    """A copy of ``t`` when its data does not start on a 16-byte boundary (the gate kernels move
    16-byte chunks).  Views into a larger tensor, such as the q / k / v that ``x.split(H, dim=1)``
    gives at B = 1 with an odd H * L, may start anywhere."""
    return t if t.data_ptr() % 16 == 0 else t.clone()


def gate_code(gate) -> int:
    """``"identity" | "sigmoid" | "silu"`` or an ``nn.Identity / nn.Sigmoid / nn.SiLU`` instance -> C gate code."""
    if isinstance(gate, str):
        try:
            return GATE_CODES[gate.strip().lower()]
        except KeyError as exc:
            raise ValueError(f"unknown gate {gate!r}; expected one of {sorted(GATE_CODES)}") from exc
    for cls, code in _MODULE_CODES.items():
        if type(gate) is cls:
            return code
    raise NotImplementedError(
        f"fft_backend='hip' fuses only Identity, Sigmoid and SiLU gates; got {type(gate).__name__}")


def gated_causal_fftconv1d_fwd_raw(q, kg, v, k, s, y, y1, act1: int, act2: int, kbatch: int = 1):
    """Launch the gated forward: q, kg, v, y, y1 ``[B, H, L]`` (y1 may be None), k ``[kbatch*H, K]`` fp32."""
    lib = _lib.get_lib()
    _lib.check_device(q)
    B, H, L = q.shape
    K = k.shape[-1]
    dt = _lib.dtype_code(q.dtype)
    need = lib.nsq_gated_fftconv1d_causal_workspace_bytes(B, H, L, K, kbatch, dt, _lib.NSQ_DIR_FWD)
    ws = _workspace(q.device, need)
    _lib.check(lib.nsq_gated_fftconv1d_causal_fwd(
        q.data_ptr(), kg.data_ptr(), v.data_ptr(), k.data_ptr(), _lib.ptr(s), y.data_ptr(), _lib.ptr(y1), dt, act1,
        act2, B, H, L, K, kbatch, _lib.ptr(ws), 0 if ws is None else ws.numel(), _lib.stream_ptr(q.device)))
    return y


def gated_causal_fftconv1d_bwd_raw(g, q, kg, v, y1, k, s, dq, dkg, dv, gk, gs, act1: int, act2: int,
                                   kbatch: int = 1):
    """Launch the gated backward (gk ``[kbatch*H, K]``, gs ``[kbatch*H]`` partials or None): elementwise gate
    kernels around the plain conv adjoint."""
    lib = _lib.get_lib()
    _lib.check_device(q)
    B, H, L = q.shape
    K = k.shape[-1]
    dt = _lib.dtype_code(q.dtype)
    need = lib.nsq_gated_fftconv1d_causal_workspace_bytes(B, H, L, K, kbatch, dt, _lib.NSQ_DIR_BWD)
    ws = _workspace(q.device, need)
    _lib.check(lib.nsq_gated_fftconv1d_causal_bwd(
        g.data_ptr(), q.data_ptr(), kg.data_ptr(), v.data_ptr(), y1.data_ptr(), k.data_ptr(), _lib.ptr(s),
        dq.data_ptr(), dkg.data_ptr(), dv.data_ptr(), gk.data_ptr(), _lib.ptr(gs), dt, act1, act2, B, H, L, K, kbatch,
        0, _lib.ptr(ws), 0 if ws is None else ws.numel(), _lib.stream_ptr(q.device)))


def _grad_wanted(*ts) -> bool:
    return torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in ts)


def _shortcut_grad(gs, s, kbatch, H):
    if s is None:
        return None
    return (gs if kbatch == 1 else gs.view(kbatch, H).sum(0)).to(s.dtype)


@custom_op("nsq_hip::gated_causal_fftconv1d", mutates_args=())
def gated_causal_fftconv1d_op(q: torch.Tensor, kg: torch.Tensor, v: torch.Tensor, k: torch.Tensor,
                              s: Optional[torch.Tensor], act1: int, act2: int, kbatch: int,
                              keep: bool) -> tuple[torch.Tensor, torch.Tensor]:
    """Gated causal conv forward; returns ``(y, y1)``, y1 = conv(z) + s z kept for the backward when ``keep``
    (else empty)."""
    q, kg, v = (_aligned16(t) for t in (q, kg, v))
    y = torch.empty_like(q)
    y1 = torch.empty_like(q) if keep else q.new_empty(0)
    gated_causal_fftconv1d_fwd_raw(q, kg, v, k, s, y, y1 if keep else None, act1, act2, kbatch)
    return y, y1


@gated_causal_fftconv1d_op.register_fake
def _(q, kg, v, k, s, act1, act2, kbatch, keep):
    return torch.empty_like(q), (torch.empty_like(q) if keep else q.new_empty(0))


@custom_op("nsq_hip::gated_causal_fftconv1d_backward", mutates_args=())
def gated_causal_fftconv1d_backward_op(g: torch.Tensor, q: torch.Tensor, kg: torch.Tensor, v: torch.Tensor,
                                       y1: torch.Tensor, k: torch.Tensor, s: Optional[torch.Tensor], act1: int,
                                       act2: int, kbatch: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor,
                                                                        torch.Tensor, torch.Tensor]:
    """``(dq, dkg, dv, gk, gs)``; gs ``[kbatch*H]`` partials, empty without a shortcut."""
    g, q, kg, v = (_aligned16(t) for t in (g, q, kg, v))
    dq, dkg, dv = torch.empty_like(q), torch.empty_like(q), torch.empty_like(q)
    gk = torch.empty_like(k)
    gs = torch.empty(kbatch * q.shape[1] if s is not None else 0, dtype=torch.float32, device=q.device)
    gated_causal_fftconv1d_bwd_raw(g, q, kg, v, y1, k, s, dq, dkg, dv, gk, gs if s is not None else None, act1, act2,
                                   kbatch)
    return dq, dkg, dv, gk, gs


@gated_causal_fftconv1d_backward_op.register_fake
def _(g, q, kg, v, y1, k, s, act1, act2, kbatch):
    return (torch.empty_like(q), torch.empty_like(q), torch.empty_like(q), torch.empty_like(k),
            q.new_empty(kbatch * q.shape[1] if s is not None else 0, dtype=torch.float32))


def _gated1d_setup(ctx, inputs, output):
    q, kg, v, k, s, act1, act2, kbatch, _keep = inputs
    # the second output is internal (state kept for the backward): no gradient flows into it, and none is
    # materialized for it (autograd would otherwise fill a zero tensor of its size before every backward)
    ctx.mark_non_differentiable(output[1])
    ctx.set_materialize_grads(False)
    ctx.save_for_backward(q, kg, v, output[1], k, s)
    ctx.meta = (act1, act2, kbatch)


def _gated1d_backward(ctx, gy, _gy1):
    q, kg, v, y1, k, s = ctx.saved_tensors
    act1, act2, kbatch = ctx.meta
    g = channels_first_contiguous(gy.to(q.dtype))
    dq, dkg, dv, gk, gs = gated_causal_fftconv1d_backward_op(g, q, kg, v, y1, k, s, act1, act2, kbatch)
    return dq, dkg, dv, gk, _shortcut_grad(gs, s, kbatch, q.shape[1]), None, None, None, None


gated_causal_fftconv1d_op.register_autograd(_gated1d_backward, setup_context=_gated1d_setup)


def hyena_gated_causal_fftconv1d_bhl(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    kernel: torch.Tensor,
    shortcut: torch.Tensor | None = None,
    gate_nonlinear="silu",
    gate_nonlinear_2=None,
) -> torch.Tensor:
    """``(conv(q*act1(k)) + s*(q*act1(k))) * act2(v)`` for BHL ``[B, H, L]`` q, k, v.

    ``kernel``: ``[1|B, H, K]`` or ``[H, K]`` fp32-castable (``K <= 2L``, the causal
    conv's rule); ``shortcut``: ``[H]`` or None.  Returns ``[B, H, L]`` in
    ``query.dtype``.
    """
    if query.ndim != 3 or key.shape != query.shape or value.shape != query.shape:
        raise ValueError(f"query, key, value must share one [B, H, L] shape; got {tuple(query.shape)}, "
                         f"{tuple(key.shape)}, {tuple(value.shape)}")
    B, H, L = query.shape
    act1 = gate_code(gate_nonlinear)
    act2 = act1 if gate_nonlinear_2 is None else gate_code(gate_nonlinear_2)
    k3 = _kernel_3d(kernel, B)
    if k3.shape[1] != H:
        raise ValueError(f"kernel has {k3.shape[1]} channels, query has {H}")
    if k3.shape[-1] > 2 * L:
        raise ValueError(f"Kernel length must be less than or equal to 2 * seq_len. Got {k3.shape[-1]}.")
    kbatch = k3.shape[0]
    in_dtype = query.dtype
    cdt = in_dtype if in_dtype in _lib.NSQ_DTYPE else torch.float32
    q, kg, v = (channels_first_contiguous(t.to(cdt)) for t in (query, key, value))
    kc = channels_first_contiguous(k3.float()).reshape(kbatch * H, k3.shape[-1])
    sc = None
    if shortcut is not None:
        if shortcut.shape != (H,):
            raise ValueError(f"shortcut must have shape ({H},); got {tuple(shortcut.shape)}")
        sc = shortcut.to(in_dtype).to(cdt).contiguous()
    y, _ = gated_causal_fftconv1d_op(q, kg, v, kc, sc, act1, act2, kbatch, _grad_wanted(q, kg, v, kc, sc))
    return y.to(in_dtype)


# ---------------------------------------------------------------------------
# 2D / 3D (nsq_gated_fftconv_nd_*): the gates inside the N-d conv's first and last passes (packed 2D rows
# with the vector epilogue, 3D plane passes), else the gate kernels around it
# ---------------------------------------------------------------------------
def _gated_nd_ws(q, k, kbatch, periodic, direction):
    lib = _lib.get_lib()
    nd = q.ndim - 2
    return int(lib.nsq_gated_fftconv_nd_workspace_bytes(
        nd, int(q.shape[0]), int(q.shape[1]), _lib.i64_array([int(d) for d in q.shape[2:]]),
        _lib.i64_array([int(d) for d in k.shape[1:]]), kbatch, periodic, _lib.dtype_code(q.dtype), direction))


@custom_op("nsq_hip::gated_fftconv_nd", mutates_args=())
def gated_fftconv_nd_op(q: torch.Tensor, kg: torch.Tensor, v: torch.Tensor, k: torch.Tensor,
                        s: Optional[torch.Tensor], act1: int, act2: int, kbatch: int, periodic: int,
                        keep: bool) -> tuple[torch.Tensor, torch.Tensor]:
    """Gated 2D/3D conv forward: q, kg, v ``[B, H, *S]`` contiguous, k ``[kbatch*H, *K]`` float32, s ``[H]`` or None;
    returns ``(y, y1)`` with y1 kept when ``keep`` (else empty)."""
    lib = _lib.get_lib()
    _lib.check_device(q)
    nd = q.ndim - 2
    B, H = q.shape[:2]
    S, K = _lib.i64_array(q.shape[2:]), _lib.i64_array(k.shape[1:])
    dt = _lib.dtype_code(q.dtype)
    q, kg, v = (_aligned16(t) for t in (q, kg, v))
    y = torch.empty_like(q)
    y1 = torch.empty_like(q) if keep else q.new_empty(0)
    ws = _workspace(q.device, _gated_nd_ws(q, k, kbatch, periodic, _lib.NSQ_DIR_FWD))
    _lib.check(lib.nsq_gated_fftconv_nd_fwd(
        nd, q.data_ptr(), kg.data_ptr(), v.data_ptr(), k.data_ptr(), _lib.ptr(s), y.data_ptr(),
        y1.data_ptr() if keep else None, dt, act1, act2, B, H, S, K, kbatch, periodic, _lib.ptr(ws),
        0 if ws is None else ws.numel(), _lib.stream_ptr(q.device)))
    return y, y1


@gated_fftconv_nd_op.register_fake
def _(q, kg, v, k, s, act1, act2, kbatch, periodic, keep):
    return torch.empty_like(q), (torch.empty_like(q) if keep else q.new_empty(0))


@custom_op("nsq_hip::gated_fftconv_nd_backward", mutates_args=())
def gated_fftconv_nd_backward_op(g: torch.Tensor, q: torch.Tensor, kg: torch.Tensor, v: torch.Tensor,
                                 y1: torch.Tensor, k: torch.Tensor, s: Optional[torch.Tensor], act1: int, act2: int,
                                 kbatch: int, periodic: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor,
                                                                      torch.Tensor, torch.Tensor]:
    """``(dq, dkg, dv, gk, gs)``; gs ``[kbatch*H]`` partials, empty without a shortcut."""
    lib = _lib.get_lib()
    nd = q.ndim - 2
    B, H = q.shape[:2]
    S, K = _lib.i64_array(q.shape[2:]), _lib.i64_array(k.shape[1:])
    dt = _lib.dtype_code(q.dtype)
    g, q, kg, v = (_aligned16(t) for t in (g, q, kg, v))
    dq, dkg, dv = torch.empty_like(q), torch.empty_like(q), torch.empty_like(q)
    gk = torch.empty_like(k)
    gs = torch.empty(kbatch * H if s is not None else 0, dtype=torch.float32, device=q.device)
    ws = _workspace(q.device, _gated_nd_ws(q, k, kbatch, periodic, _lib.NSQ_DIR_BWD))
    _lib.check(lib.nsq_gated_fftconv_nd_bwd(
        nd, g.data_ptr(), q.data_ptr(), kg.data_ptr(), v.data_ptr(), y1.data_ptr(), k.data_ptr(), _lib.ptr(s),
        dq.data_ptr(), dkg.data_ptr(), dv.data_ptr(), gk.data_ptr(), gs.data_ptr() if s is not None else None, dt,
        act1, act2, B, H, S, K, kbatch, periodic, _lib.ptr(ws), 0 if ws is None else ws.numel(),
        _lib.stream_ptr(q.device)))
    return dq, dkg, dv, gk, gs


@gated_fftconv_nd_backward_op.register_fake
def _(g, q, kg, v, y1, k, s, act1, act2, kbatch, periodic):
    return (torch.empty_like(q), torch.empty_like(q), torch.empty_like(q), torch.empty_like(k),
            q.new_empty(kbatch * q.shape[1] if s is not None else 0, dtype=torch.float32))


def _gatednd_setup(ctx, inputs, output):
    q, kg, v, k, s, act1, act2, kbatch, periodic, _keep = inputs
    # the second output is internal (state kept for the backward): no gradient flows into it, and none is
    # materialized for it (autograd would otherwise fill a zero tensor of its size before every backward)
    ctx.mark_non_differentiable(output[1])
    ctx.set_materialize_grads(False)
    ctx.save_for_backward(q, kg, v, output[1], k, s)
    ctx.meta = (act1, act2, kbatch, periodic)


def _gatednd_backward(ctx, gy, _gy1):
    q, kg, v, y1, k, s = ctx.saved_tensors
    act1, act2, kbatch, periodic = ctx.meta
    g = channels_first_contiguous(gy.to(q.dtype))
    dq, dkg, dv, gk, gs = gated_fftconv_nd_backward_op(g, q, kg, v, y1, k, s, act1, act2, kbatch, periodic)
    return dq, dkg, dv, gk, _shortcut_grad(gs, s, kbatch, q.shape[1]), None, None, None, None, None


gated_fftconv_nd_op.register_autograd(_gatednd_backward, setup_context=_gatednd_setup)


def hyena_gated_fftconv_nd_bhl(query, key, value, kernel, shortcut=None, gate_nonlinear="silu",
                               gate_nonlinear_2=None, periodic=None) -> torch.Tensor:
    """``(conv(q*act1(k)) + s*(q*act1(k))) * act2(v)`` for ``[B, H, *S]`` q, k, v (2D or 3D), with the
    non-causal N-d conv of CKConvND: ``periodic`` per axis (None = all zero-padded "same").

    ``kernel``: ``[1|B, H, *K]`` or ``[H, *K]`` (``K_d <= 2 S_d`` zero-padded, ``K_d <= S_d`` periodic);
    ``shortcut``: ``[H]`` or None.  Returns ``query.dtype``.
    """
    if query.ndim not in (4, 5) or key.shape != query.shape or value.shape != query.shape:
        raise ValueError(f"query, key, value must share one [B, H, *S] shape (2D or 3D); got {tuple(query.shape)}, "
                         f"{tuple(key.shape)}, {tuple(value.shape)}")
    nd = query.ndim - 2
    B, H = query.shape[:2]
    per = (False,) * nd if periodic is None else tuple(bool(p) for p in periodic)
    if len(per) != nd:
        raise ValueError(f"periodic must have {nd} entries; got {per}")
    act1 = gate_code(gate_nonlinear)
    act2 = act1 if gate_nonlinear_2 is None else gate_code(gate_nonlinear_2)
    k = kernel if kernel.ndim == nd + 2 else kernel.unsqueeze(0)
    if k.ndim != nd + 2 or k.shape[0] not in (1, B) or k.shape[1] != H:
        raise ValueError(f"kernel must be [1|B, H, *K] or [H, *K]; got {tuple(kernel.shape)}")
    kbatch = k.shape[0]
    in_dtype = query.dtype
    cdt = in_dtype if in_dtype in _lib.NSQ_DTYPE else torch.float32
    q, kg, v = (channels_first_contiguous(t.to(cdt)) for t in (query, key, value))
    kc = channels_first_contiguous(k.float()).reshape(kbatch * H, *k.shape[2:])
    sc = None
    if shortcut is not None:
        if shortcut.shape != (H,):
            raise ValueError(f"shortcut must have shape ({H},); got {tuple(shortcut.shape)}")
        sc = shortcut.to(in_dtype).to(cdt).contiguous()
    if needs_extension(q.shape[2:], per):
        # a periodic axis of a length the periodic plans do not take: the gates as the reference computes them
        # (hyena_nd.py:546,570) around the conv on the periodic extension
        z = q * _TORCH_GATES[act1](kg)
        y1 = periodic_by_extension(z, kc.view(kbatch, H, *kc.shape[1:]), sc, per)
        return (y1 * _TORCH_GATES[act2](v)).to(in_dtype)
    y, _ = gated_fftconv_nd_op(q, kg, v, kc, sc, act1, act2, kbatch, periodic_mask(per), _grad_wanted(q, kg, v, kc, sc))
    return y.to(in_dtype)


def hyena_gated_fftconv2d_bhl(query, key, value, kernel, shortcut=None, gate_nonlinear="silu",
                              gate_nonlinear_2=None, periodic=None) -> torch.Tensor:
    """2D form of :func:`hyena_gated_fftconv_nd_bhl` (``[B, H, X, Y]``)."""
    if query.ndim != 4:
        raise ValueError(f"expected [B, H, X, Y]; got {tuple(query.shape)}")
    return hyena_gated_fftconv_nd_bhl(query, key, value, kernel, shortcut, gate_nonlinear, gate_nonlinear_2, periodic)


def hyena_gated_fftconv3d_bhl(query, key, value, kernel, shortcut=None, gate_nonlinear="silu",
                              gate_nonlinear_2=None, periodic=None) -> torch.Tensor:
    """3D form of :func:`hyena_gated_fftconv_nd_bhl` (``[B, H, X, Y, Z]``)."""
    if query.ndim != 5:
        raise ValueError(f"expected [B, H, X, Y, Z]; got {tuple(query.shape)}")
    return hyena_gated_fftconv_nd_bhl(query, key, value, kernel, shortcut, gate_nonlinear, gate_nonlinear_2, periodic)
