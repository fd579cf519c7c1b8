r"""Hyena-gated causal 1D FFT convolution on the HIP backend (build-plan row F2).

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
plain conv adjoint by default; the one-kernel gated adjoint
(``fuse_backward_gates=True``) measured slower on MI355X (a latency-bound kernel
at one workgroup per CU gains five operand streams).  Gates: ``"identity"``, ``"sigmoid"``, ``"silu"`` or the
matching ``torch.nn`` modules; ``gate_nonlinear_2=None`` reuses the first gate,
as ``Hyena.__init__`` does (``hyena_nd.py:274-278``).  Results follow the
reference composition with each elementwise product rounded to the I/O dtype.
"""

from __future__ import annotations

import torch

from . import _lib
from .fftconv_hip import _kernel_3d, _workspace
from .mixed_fftconv_hip import periodic_mask


__all__ = ["GATE_CODES", "gate_code", "hyena_gated_causal_fftconv1d_bhl", "gated_causal_fftconv1d_fwd_raw",
           "gated_causal_fftconv1d_bwd_raw", "hyena_gated_fftconv2d_bhl", "hyena_gated_fftconv3d_bhl",
           "hyena_gated_fftconv_nd_bhl"]

GATE_CODES = {"identity": 0, "sigmoid": 1, "silu": 2}
_MODULE_CODES = {torch.nn.Identity: 0, torch.nn.Sigmoid: 1, torch.nn.SiLU: 2}


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
                                   kbatch: int = 1, fuse_gates: bool = False):
    """Launch the gated backward (gk ``[kbatch*H, K]``, gs ``[kbatch*H]`` partials or None).

    ``fuse_gates``: the one-kernel adjoint with the gates inside (FFT lengths <= 16384); the default runs
    the elementwise gate kernels around the plain adjoint, measured faster on MI355X."""
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
        int(bool(fuse_gates)), _lib.ptr(ws), 0 if ws is None else ws.numel(), _lib.stream_ptr(q.device)))


class _GatedCausalFFTConv1d(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, kg, v, k, s, act1, act2, kbatch, fuse_bwd=False):
        y = torch.empty_like(q)
        keep = any(ctx.needs_input_grad[:5])
        y1 = torch.empty_like(q) if keep else None
        gated_causal_fftconv1d_fwd_raw(q, kg, v, k, s, y, y1, act1, act2, kbatch)
        ctx.save_for_backward(q, kg, v, y1, k, s)
        ctx.acts = (act1, act2)
        ctx.kbatch = kbatch
        ctx.fuse_bwd = fuse_bwd
        ctx.has_s = s is not None
        return y

    @staticmethod
    def backward(ctx, gy):
        q, kg, v, y1, k, s = ctx.saved_tensors
        g = _aligned16(gy.to(q.dtype).contiguous())
        dq, dkg, dv = torch.empty_like(q), torch.empty_like(q), torch.empty_like(q)
        gk = torch.empty_like(k)
        H = q.shape[1]
        gs = torch.empty(ctx.kbatch * H, dtype=torch.float32, device=q.device) if ctx.has_s else None
        gated_causal_fftconv1d_bwd_raw(g, q, kg, v, y1, k, s, dq, dkg, dv, gk, gs, *ctx.acts, ctx.kbatch, ctx.fuse_bwd)
        gsum = None
        if ctx.has_s:
            gsum = (gs if ctx.kbatch == 1 else gs.view(ctx.kbatch, H).sum(0)).to(s.dtype)
        return dq, dkg, dv, gk, gsum, None, None, None, None


def hyena_gated_causal_fftconv1d_bhl(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    kernel: torch.Tensor,
    shortcut: torch.Tensor | None = None,
    gate_nonlinear="silu",
    gate_nonlinear_2=None,
    fuse_backward_gates: bool = False,
) -> torch.Tensor:
    """``(conv(q*act1(k)) + s*(q*act1(k))) * act2(v)`` for BHL ``[B, H, L]`` q, k, v.

    ``kernel``: ``[1|B, H, K]`` or ``[H, K]`` fp32-castable (``K <= 2L``, the causal
    conv's rule); ``shortcut``: ``[H]`` or None.  Returns ``[B, H, L]`` in
    ``query.dtype``.  ``fuse_backward_gates``: run the backward's gates inside the
    fused adjoint too (FFT lengths <= 16384; slower on MI355X at the measured shapes).
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
    q, kg, v = (_aligned16(t.to(cdt).contiguous()) for t in (query, key, value))
    kc = k3.float().reshape(kbatch * H, k3.shape[-1]).contiguous()
    sc = None
    if shortcut is not None:
        if shortcut.shape != (H,):
            raise ValueError(f"shortcut must have shape ({H},); got {tuple(shortcut.shape)}")
        sc = shortcut.to(in_dtype).to(cdt).contiguous()
    return _GatedCausalFFTConv1d.apply(q, kg, v, kc, sc, act1, act2, kbatch, fuse_backward_gates).to(in_dtype)


# ---------------------------------------------------------------------------
# 2D / 3D: the gate kernels around the N-d conv (nsq_gated_fftconv_nd_*)
# ---------------------------------------------------------------------------
class _GatedFFTConvND(torch.autograd.Function):
    """q, kg, v: [B, H, *S] contiguous; k: [kbatch*H, *K] contiguous float32; s: [H] or None."""

    @staticmethod
    def forward(ctx, q, kg, v, k, s, act1, act2, kbatch, periodic):
        lib = _lib.get_lib()
        _lib.check_device(q)
        nd = q.ndim - 2
        B, H = q.shape[:2]
        S, K = _lib.i64_array(q.shape[2:]), _lib.i64_array(k.shape[1:])
        dt = _lib.dtype_code(q.dtype)
        y = torch.empty_like(q)
        keep = any(ctx.needs_input_grad[:5])
        y1 = torch.empty_like(q) if keep else None
        ws = _workspace(q.device, lib.nsq_gated_fftconv_nd_workspace_bytes(nd, B, H, S, K, kbatch, periodic, dt,
                                                                            _lib.NSQ_DIR_FWD))
        _lib.check(lib.nsq_gated_fftconv_nd_fwd(
            nd, q.data_ptr(), kg.data_ptr(), v.data_ptr(), k.data_ptr(), _lib.ptr(s), y.data_ptr(), _lib.ptr(y1), dt,
            act1, act2, B, H, S, K, kbatch, periodic, _lib.ptr(ws), 0 if ws is None else ws.numel(),
            _lib.stream_ptr(q.device)))
        ctx.save_for_backward(q, kg, v, y1, k, s)
        ctx.meta = (act1, act2, kbatch, periodic)
        ctx.has_s = s is not None
        return y

    @staticmethod
    def backward(ctx, gy):
        q, kg, v, y1, k, s = ctx.saved_tensors
        act1, act2, kbatch, periodic = ctx.meta
        lib = _lib.get_lib()
        nd = q.ndim - 2
        B, H = q.shape[:2]
        S, K = _lib.i64_array(q.shape[2:]), _lib.i64_array(k.shape[1:])
        dt = _lib.dtype_code(q.dtype)
        g = _aligned16(gy.to(q.dtype).contiguous())
        dq, dkg, dv = torch.empty_like(q), torch.empty_like(q), torch.empty_like(q)
        gk = torch.empty_like(k)
        gs = torch.empty(kbatch * H, dtype=torch.float32, device=q.device) if ctx.has_s else None
        ws = _workspace(q.device, lib.nsq_gated_fftconv_nd_workspace_bytes(nd, B, H, S, K, kbatch, periodic, dt,
                                                                            _lib.NSQ_DIR_BWD))
        _lib.check(lib.nsq_gated_fftconv_nd_bwd(
            nd, g.data_ptr(), q.data_ptr(), kg.data_ptr(), v.data_ptr(), y1.data_ptr(), k.data_ptr(), _lib.ptr(s),
            dq.data_ptr(), dkg.data_ptr(), dv.data_ptr(), gk.data_ptr(), _lib.ptr(gs), dt, act1, act2, B, H, S, K,
            kbatch, periodic, _lib.ptr(ws), 0 if ws is None else ws.numel(), _lib.stream_ptr(q.device)))
        gsum = None
        if ctx.has_s:
            gsum = (gs if kbatch == 1 else gs.view(kbatch, H).sum(0)).to(s.dtype)
        return dq, dkg, dv, gk, gsum, None, None, None, None


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
    q, kg, v = (_aligned16(t.to(cdt).contiguous()) for t in (query, key, value))
    kc = k.float().reshape(kbatch * H, *k.shape[2:]).contiguous()
    sc = None
    if shortcut is not None:
        if shortcut.shape != (H,):
            raise ValueError(f"shortcut must have shape ({H},); got {tuple(shortcut.shape)}")
        sc = shortcut.to(in_dtype).to(cdt).contiguous()
    return _GatedFFTConvND.apply(q, kg, v, kc, sc, act1, act2, kbatch, periodic_mask(per)).to(in_dtype)


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
