r"""HIP (gfx950) FFT long-convolution ops with the ``nvsubquadratic.ops`` call signatures.

This module is the ``fft_backend="hip"`` counterpart of the reference's
``nvsubquadratic/ops/fftconv_custom.py`` (the ``"subq_ops"`` backend).  Every
public function keeps the reference name, argument order, accepted shapes,
dtype behaviour and error types, so a caller switches backends by changing the
import (or ``CKConvND(fft_backend=...)``, see :mod:`nvsubquadratic_amd.dispatch`).

Semantics (reference ``nvsubquadratic/ops/fftconv_custom.py:307-335`` on top of
``nvsubquadratic/ops/fftconv.py:546-600``):

* the op accepts any input dtype, computes in float32 and returns ``x.dtype``;
* ``y = conv(x, kernel).to(x.dtype)``, then ``y = y + shortcut.to(x.dtype) * x``;
* 1D kernels: shared ``[1, H, K]`` / ``[H, K]``, or per-sample (FiLM)
  ``[B, H, K]``.  The reference's native wrapper raises ``NotImplementedError``
  for the latter (``fftconv_custom.py:294-300``); its torch path accepts it
  (``fftconv.py:546-600``), and so does this backend, with that path's results.

Differences in *how*: the whole chain (pad, real FFT, spectral product,
inverse FFT, crop, cast and shortcut) runs inside hand-written HIP kernels
(``csrc/fftconv1d.hip``) with a fused backward; nothing is computed on the CPU.
"""

from __future__ import annotations

from typing import Optional

import os

import torch
from einops import rearrange
from torch.library import custom_op

from . import _lib
from .layout import channels_first_contiguous


__all__ = [
    "causal_fftconv1d_bhl",
    "causal_fftconv1d_bhl_chunked",
    "causal_fftconv1d_bhl_w_reshape",
    "causal_fftconv1d_bhl_w_reshape_chunked",
    "causal_fftconv1d_blh",
    "causal_fftconv1d_blh_chunked",
    "causal_fftconv1d_fwd_raw",
    "causal_fftconv1d_bwd_raw",
    "fftconv1d_bhl",
    "fftconv1d_bhl_chunked",
    "fftconv1d_bhl_w_reshape",
    "fftconv1d_bhl_w_reshape_chunked",
    "fftconv1d_blh",
    "fftconv1d_blh_chunked",
    "mixed_fftconv1d_fwd_raw",
    "mixed_fftconv1d_bwd_raw",
    "fftconv2d_bhl",
    "fftconv2d_bhl_chunked",
    "fftconv2d_bhl_w_reshape",
    "fftconv2d_bhl_w_reshape_chunked",
    "fftconv2d_blh",
    "fftconv2d_blh_chunked",
    "fftconv3d_bhl",
    "fftconv3d_bhl_chunked",
    "fftconv3d_bhl_w_reshape",
    "fftconv3d_bhl_w_reshape_chunked",
    "fftconv3d_blh",
    "fftconv3d_blh_chunked",
    "fftconv_nd_bwd_raw",
    "fftconv_nd_fwd_raw",
]

_DEFAULT_CHUNK_SIZE = 128


# ---------------------------------------------------------------------------
# Raw launches (preallocated outputs; used by the custom ops below, tests and bench)
# ---------------------------------------------------------------------------
def _workspace(device: torch.device, nbytes: int) -> torch.Tensor | None:
    if nbytes == 0:
        return None
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


def _causal_workspace_bytes(lib, B, H, L, K, kbatch, direction):
    if kbatch != 1:
        return lib.nsq_fftconv1d_causal_film_workspace_bytes(B, H, L, K, kbatch, direction)
    return lib.nsq_fftconv1d_causal_workspace_bytes(B, H, L, K, direction)


def causal_fftconv1d_fwd_raw(
    x: torch.Tensor,
    k: torch.Tensor,
    s: torch.Tensor | None,
    y: torch.Tensor,
    workspace: torch.Tensor | None = None,
    kbatch: int = 1,
) -> torch.Tensor:
    """Launch the forward kernel on the current stream.

    ``x``/``y``: contiguous ``[B, H, L]`` (float32/bfloat16/float16, same dtype);
    ``k``: contiguous float32 ``[kbatch*H, K]`` (kbatch 1, or B for per-sample
    filters); ``s``: ``[H]`` in ``x.dtype`` or None.
    """
    lib = _lib.get_lib()
    _lib.check_device(x)
    B, H, L = x.shape
    K = k.shape[-1]
    need = _causal_workspace_bytes(lib, B, H, L, K, kbatch, _lib.NSQ_DIR_FWD)
    if need and (workspace is None or workspace.numel() < need):
        workspace = _workspace(x.device, need)
    args = (x.data_ptr(), k.data_ptr(), _lib.ptr(s), y.data_ptr(), _lib.dtype_code(x.dtype), B, H, L, K)
    tail = (_lib.ptr(workspace), 0 if workspace is None else workspace.numel(), _lib.stream_ptr(x.device))
    if kbatch != 1:
        rc = lib.nsq_fftconv1d_causal_film_fwd(*args, kbatch, *tail)
    else:
        rc = lib.nsq_fftconv1d_causal_fwd(*args, *tail)
    _lib.check(rc)
    return y


def causal_fftconv1d_bwd_raw(
    g: torch.Tensor,
    x: torch.Tensor,
    k: torch.Tensor,
    s: torch.Tensor | None,
    gx: torch.Tensor,
    gk: torch.Tensor,
    gs: torch.Tensor | None,
    workspace: torch.Tensor | None = None,
    fwd_state: bool = False,
    kbatch: int = 1,
) -> None:
    """Launch the backward kernels on the current stream (see include/nsq_hip.h).

    ``fwd_state=True`` reuses the transformed x and k that a forward call left
    in ``workspace`` (a forward given a workspace of the backward's size keeps
    them); the workspace must be untouched since that forward.  Per-sample
    filters (``kbatch = B``): gk ``[B*H, K]``, gs ``[B*H]`` partials.
    """
    lib = _lib.get_lib()
    _lib.check_device(x)
    B, H, L = x.shape
    K = k.shape[-1]
    need = _causal_workspace_bytes(lib, B, H, L, K, kbatch, _lib.NSQ_DIR_BWD)
    if need and (workspace is None or workspace.numel() < need):
        workspace = _workspace(x.device, need)
        fwd_state = False
    args = (g.data_ptr(), x.data_ptr(), k.data_ptr(), _lib.ptr(s), gx.data_ptr(), gk.data_ptr(), _lib.ptr(gs),
            _lib.dtype_code(x.dtype), B, H, L, K)
    tail = (_lib.ptr(workspace), 0 if workspace is None else workspace.numel(), int(bool(fwd_state)),
            _lib.stream_ptr(x.device))
    if kbatch != 1:
        rc = lib.nsq_fftconv1d_causal_film_bwd(*args, kbatch, *tail)
    else:
        rc = lib.nsq_fftconv1d_causal_bwd(*args, *tail)
    _lib.check(rc)


# ---------------------------------------------------------------------------
# Operators.  Every HIP op is a torch.library custom op (namespace nsq_hip) with
# a fake (meta) implementation and a registered autograd formula, so that
# torch.compile traces through it (fullgraph) instead of breaking the graph at
# an opaque ctypes call; eager calls dispatch to the same implementations.
# ---------------------------------------------------------------------------
def _grad_wanted(*ts) -> bool:
    return torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in ts)


def state_budget_bytes(device: torch.device) -> int:
    """Largest forward state (transformed x and filter, kept for the backward) one call keeps.

    ``NSQ_STATE_MAX_BYTES`` (bytes) sets it; by default an eighth of the device's memory (36 GB on one
    MI355X: config 3's 24 GiB is kept).  A larger state is not kept and the backward recomputes the
    transforms from x and the filter (config 3: two more column passes, ~4.5 ms)."""
    env = os.environ.get("NSQ_STATE_MAX_BYTES")
    if env is not None:
        return int(env)
    if device.type != "cuda" or not torch.cuda.is_available():  # shape propagation without a GPU
        return 1 << 62
    return torch.cuda.get_device_properties(device).total_memory // 8




def _within_budget(nbytes: int, device: torch.device) -> int:
    """``nbytes`` if that state fits :func:`state_budget_bytes`, else 0 (no state kept)."""
    return nbytes if nbytes <= state_budget_bytes(device) else 0


def _causal_state_bytes(x: torch.Tensor, k: torch.Tensor, kbatch: int, keep: bool) -> int:
    if not keep:
        return 0
    B, H, L = (int(d) for d in x.shape)
    return _within_budget(
        int(_causal_workspace_bytes(_lib.get_lib(), B, H, L, int(k.shape[-1]), kbatch, _lib.NSQ_DIR_BWD)), x.device)


@custom_op("nsq_hip::causal_fftconv1d", mutates_args=())
def causal_fftconv1d_op(x: torch.Tensor, k: torch.Tensor, s: Optional[torch.Tensor], kbatch: int,
                        keep: bool) -> tuple[torch.Tensor, torch.Tensor]:
    """Causal FFT conv forward; x ``[B, H, L]`` contiguous (f32/bf16/f16), k ``[kbatch*H, K]`` float32, s ``[H]``
    in x.dtype or None.  Returns ``(y, state)``: with ``keep`` the state is a backward-sized workspace in which the
    forward leaves its transformed x and k for the backward (like autograd keeping rfft outputs), else empty."""
    y = torch.empty_like(x)
    state = torch.empty(_causal_state_bytes(x, k, kbatch, keep), dtype=torch.uint8, device=x.device)
    causal_fftconv1d_fwd_raw(x, k, s, y, state if state.numel() else None, kbatch)
    return y, state


@causal_fftconv1d_op.register_fake
def _(x, k, s, kbatch, keep):
    return torch.empty_like(x), x.new_empty(_causal_state_bytes(x, k, kbatch, keep), dtype=torch.uint8)


@custom_op("nsq_hip::causal_fftconv1d_backward", mutates_args=("state",))
def causal_fftconv1d_backward_op(g: torch.Tensor, x: torch.Tensor, k: torch.Tensor, s: Optional[torch.Tensor],
                                 state: torch.Tensor, kbatch: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Gradients ``(gx, gk, gs)`` (gs ``[kbatch*H]`` partial sums, empty without a shortcut); a non-empty ``state``
    is the forward's workspace and is consumed (overwritten)."""
    gx = torch.empty_like(x)
    gk = torch.empty(k.shape, dtype=torch.float32, device=x.device)
    gs = torch.empty(k.shape[0] if s is not None else 0, dtype=torch.float32, device=x.device)
    has = state.numel() > 0
    causal_fftconv1d_bwd_raw(g, x, k, s, gx, gk, gs if s is not None else None, state if has else None,
                             fwd_state=has, kbatch=kbatch)
    return gx, gk, gs


@causal_fftconv1d_backward_op.register_fake
def _(g, x, k, s, state, kbatch):
    return (torch.empty_like(x), k.new_empty(k.shape, dtype=torch.float32),
            x.new_empty(k.shape[0] if s is not None else 0, dtype=torch.float32))


def _shortcut_grad(gs: torch.Tensor, s: torch.Tensor | None, kbatch: int, H: int):
    """Per-filter partial shortcut gradients (per-sample filters) summed to ``[H]``, in the shortcut's dtype."""
    if s is None:
        return None
    return (gs if kbatch == 1 else gs.view(kbatch, H).sum(0)).to(s.dtype)


def _causal_setup(ctx, inputs, output):
    x, k, s, kbatch, _keep = inputs
    # the second output is internal (state kept for the backward): no gradient flows into it, and none is
    # materialized for it (autograd would otherwise fill a zero tensor of its size before every backward)
    ctx.mark_non_differentiable(output[1])
    ctx.set_materialize_grads(False)
    ctx.save_for_backward(x, k, s)
    ctx.state = output[1]
    ctx.kbatch = kbatch


def _take_state(ctx) -> torch.Tensor:
    """The forward's state for this backward.  The backward consumes it (overwrites it in place), so a second
    backward through the same graph (``retain_graph=True``) gets an empty state and recomputes the transforms.  The
    state is kept on ctx, not saved: the in-place use would fail saved-tensor version checks."""
    state = ctx.state
    ctx.state = state.new_empty(0)
    return state


def _causal_backward(ctx, gy, _gstate):
    x, k, s = ctx.saved_tensors
    state = _take_state(ctx)
    g = channels_first_contiguous(gy.to(x.dtype))
    gx, gk, gs = causal_fftconv1d_backward_op(g, x, k, s, state, ctx.kbatch)
    return gx, gk, _shortcut_grad(gs, s, ctx.kbatch, x.shape[1]), None, None


causal_fftconv1d_op.register_autograd(_causal_backward, setup_context=_causal_setup)


# ---------------------------------------------------------------------------
# Argument normalisation shared by every public function
# ---------------------------------------------------------------------------
def _kernel_3d(kernel: torch.Tensor, B: int) -> torch.Tensor:
    """``[H, K]`` -> ``[1, H, K]``; ``[1|B, H, K]`` kept (per-sample FiLM filters ``[B, H, K]``).

    The shape rule of ``causal_fftconv1d_fp32_bhl`` (``nvsubquadratic/ops/fftconv.py:571-574``).
    """
    if kernel.ndim == 2:
        return kernel.unsqueeze(0)
    if kernel.ndim != 3:
        raise ValueError(f"Unexpected kernel shape: {tuple(kernel.shape)}.")
    assert kernel.shape[0] in (1, B), (
        f"Leading dimension must be 1 or batch_size ({B}). Got kernel.shape={tuple(kernel.shape)}."
    )
    return kernel


def _causal_core(x: torch.Tensor, kernel: torch.Tensor, shortcut: torch.Tensor | None) -> torch.Tensor:
    if x.ndim != 3:
        raise ValueError(f"x must be [B, H, L]; got shape {tuple(x.shape)}")
    B, H, L = x.shape
    k3 = _kernel_3d(kernel, B)
    kbatch = k3.shape[0]
    if k3.shape[1] != H:
        raise ValueError(f"kernel has {k3.shape[1]} channels, x has {H}")
    if k3.shape[2] > 2 * L:
        raise ValueError(f"Kernel length must be less than or equal to 2 * seq_len. Got {k3.shape[2]}.")
    input_dtype = x.dtype
    compute_dtype = input_dtype if input_dtype in _lib.NSQ_DTYPE else torch.float32
    xc = channels_first_contiguous(x.to(compute_dtype))
    kc = channels_first_contiguous(k3.float()).reshape(kbatch * H, k3.shape[2])
    sc = None
    if shortcut is not None:
        if shortcut.shape != (H,):
            raise ValueError(f"shortcut must have shape ({H},); got {tuple(shortcut.shape)}")
        # Reference casts the shortcut to the input dtype before the product.
        sc = shortcut.to(input_dtype).to(compute_dtype).contiguous()
    y, _ = causal_fftconv1d_op(xc, kc, sc, kbatch, _grad_wanted(xc, kc, sc))
    return y.to(input_dtype)


# ---------------------------------------------------------------------------
# Public API (names and signatures of nvsubquadratic/ops/fftconv_custom.py)
# ---------------------------------------------------------------------------
def causal_fftconv1d_bhl(
    x: torch.Tensor,
    kernel: torch.Tensor,
    shortcut: torch.Tensor | None = None,
) -> torch.Tensor:
    """1D causal FFT convolution on the HIP backend, BHL layout ``[B, H, L]``.

    Drop-in for ``nvsubquadratic.ops.fftconv_custom.causal_fftconv1d_bhl``
    (``fftconv_custom.py:307-335``) and, numerically, for
    ``nvsubquadratic.ops.fftconv.causal_fftconv1d_fp32_bhl`` (``fftconv.py:546-600``).

    Args:
        x: Input ``[B, H, L]``, any floating dtype.
        kernel: ``[1, H, K]``, ``[H, K]`` or per-sample ``[B, H, K]``, with ``K <= 2L``.
        shortcut: Optional ``[H]`` per-channel scale.

    Returns:
        ``[B, H, L]`` in ``x.dtype``.
    """
    return _causal_core(x, kernel, shortcut)


def causal_fftconv1d_bhl_w_reshape(
    x: torch.Tensor,
    kernel: torch.Tensor,
    shortcut: torch.Tensor | None = None,
) -> torch.Tensor:
    """BLH inputs ``[B, L, H]`` with kernel ``[1, K, H]`` (``fftconv_custom.py:338-350``)."""
    x_bhl = rearrange(x, "b l h -> b h l")
    kernel_bhl = rearrange(kernel, "b l h -> b h l")
    y_bhl = causal_fftconv1d_bhl(x_bhl, kernel_bhl, shortcut)
    return rearrange(y_bhl, "b h l -> b l h")


def causal_fftconv1d_blh(
    x: torch.Tensor,
    kernel: torch.Tensor,
    shortcut: torch.Tensor | None = None,
) -> torch.Tensor:
    """Alias for :func:`causal_fftconv1d_bhl_w_reshape` (``fftconv_custom.py:353-359``)."""
    return causal_fftconv1d_bhl_w_reshape(x, kernel, shortcut)


def causal_fftconv1d_bhl_chunked(
    x: torch.Tensor,
    kernel: torch.Tensor,
    shortcut: torch.Tensor | None = None,
    chunk_size: int | None = None,
) -> torch.Tensor:
    """Channel-chunked variant (``fftconv_custom.py:362-389``).

    Channels are independent in every HIP kernel, so the result is bitwise
    identical to :func:`causal_fftconv1d_bhl`; chunking only bounds the size of
    the 4-step plan's workspace.
    """
    if chunk_size is None:
        chunk_size = _DEFAULT_CHUNK_SIZE
    B, H, _L = x.shape
    if H <= chunk_size:
        return causal_fftconv1d_bhl(x, kernel, shortcut)
    k3 = _kernel_3d(kernel, B)
    chunks = []
    for start in range(0, H, chunk_size):
        end = min(start + chunk_size, H)
        s_c = None if shortcut is None else shortcut[start:end]
        chunks.append(causal_fftconv1d_bhl(x[:, start:end], k3[:, start:end], s_c))
    return torch.cat(chunks, dim=1)


def causal_fftconv1d_bhl_w_reshape_chunked(
    x: torch.Tensor,
    kernel: torch.Tensor,
    shortcut: torch.Tensor | None = None,
    chunk_size: int | None = None,
) -> torch.Tensor:
    """Chunked BLH variant (``fftconv_custom.py:392-402``)."""
    x_bhl = rearrange(x, "b l h -> b h l")
    kernel_bhl = rearrange(kernel, "b l h -> b h l")
    y_bhl = causal_fftconv1d_bhl_chunked(x_bhl, kernel_bhl, shortcut, chunk_size)
    return rearrange(y_bhl, "b h l -> b l h")


def causal_fftconv1d_blh_chunked(
    x: torch.Tensor,
    kernel: torch.Tensor,
    shortcut: torch.Tensor | None = None,
    chunk_size: int | None = None,
) -> torch.Tensor:
    """Alias for :func:`causal_fftconv1d_bhl_w_reshape_chunked` (``fftconv_custom.py:405-412``)."""
    return causal_fftconv1d_bhl_w_reshape_chunked(x, kernel, shortcut, chunk_size)


# ===========================================================================
# 2D / 3D non-causal (zero-padded, "same") FFT convolution
# ===========================================================================
def _nd_workspace_bytes(lib, nd, B, H, S, K, kbatch, periodic, direction):
    if periodic:
        return lib.nsq_mixed_fftconv_nd_workspace_bytes(nd, B, H, S, K, kbatch, periodic, direction)
    return lib.nsq_fftconv_nd_workspace_bytes(nd, B, H, S, K, kbatch, direction)


def fftconv_nd_fwd_raw(x, k, s, y, kbatch: int, workspace: torch.Tensor | None = None, periodic: int = 0):
    """Launch the N-d forward on the current stream.

    ``x``/``y``: contiguous ``[B, H, *S]``; ``k``: contiguous float32
    ``[kbatch*H, *K]``; ``s``: ``[H]`` in ``x.dtype`` or None.  ``periodic``:
    bit d set = spatial axis d is circular (``nsq_mixed_fftconv_nd_fwd``);
    0 = every axis zero-padded (``nsq_fftconv_nd_fwd``).
    """
    lib = _lib.get_lib()
    _lib.check_device(x)
    nd = x.ndim - 2
    B, H = x.shape[:2]
    S = _lib.i64_array(x.shape[2:])
    K = _lib.i64_array(k.shape[1:])
    need = _nd_workspace_bytes(lib, nd, B, H, S, K, kbatch, periodic, _lib.NSQ_DIR_FWD)
    if need == 0:
        raise NotImplementedError(
            f"fft_backend='hip' {nd}D: unsupported shape x={tuple(x.shape)} k={tuple(k.shape)} periodic={periodic:#x} "
            f"(periodic axes need a power-of-two length <= 1024 and K <= S; zero-padded axes an FFT length "
            f"<= 1024)")
    if workspace is None or workspace.numel() < need:
        workspace = _workspace(x.device, need)
    args = (x.data_ptr(), k.data_ptr(), _lib.ptr(s), y.data_ptr(), _lib.dtype_code(x.dtype), B, H, S, K, kbatch)
    tail = (workspace.data_ptr(), workspace.numel(), _lib.stream_ptr(x.device))
    if periodic:
        _lib.check(lib.nsq_mixed_fftconv_nd_fwd(nd, *args, periodic, *tail))
    else:
        _lib.check(lib.nsq_fftconv_nd_fwd(nd, *args, *tail))
    return y


def fftconv_nd_bwd_raw(g, x, k, s, gx, gk, gs, kbatch: int, workspace: torch.Tensor | None = None,
                       fwd_state: bool = False, periodic: int = 0):
    """Launch the N-d backward (gs: ``[kbatch*H]`` partials or None).

    ``fwd_state=True`` reuses the transformed x and filter spectrum that a forward
    given a backward-sized ``workspace`` left there (untouched since).
    """
    lib = _lib.get_lib()
    _lib.check_device(x)
    nd = x.ndim - 2
    B, H = x.shape[:2]
    S = _lib.i64_array(x.shape[2:])
    K = _lib.i64_array(k.shape[1:])
    need = _nd_workspace_bytes(lib, nd, B, H, S, K, kbatch, periodic, _lib.NSQ_DIR_BWD)
    if workspace is None or workspace.numel() < need:
        workspace = _workspace(x.device, need)
        fwd_state = False
    args = (g.data_ptr(), x.data_ptr(), k.data_ptr(), _lib.ptr(s), gx.data_ptr(), gk.data_ptr(), _lib.ptr(gs),
            _lib.dtype_code(x.dtype), B, H, S, K, kbatch)
    tail = (workspace.data_ptr(), workspace.numel(), int(bool(fwd_state)), _lib.stream_ptr(x.device))
    if periodic:
        _lib.check(lib.nsq_mixed_fftconv_nd_bwd(nd, *args, periodic, *tail))
    else:
        _lib.check(lib.nsq_fftconv_nd_bwd(nd, *args, *tail))


def _nd_state_bytes(x: torch.Tensor, k: torch.Tensor, kbatch: int, periodic: int, keep: bool) -> int:
    if not keep:
        return 0
    nd = x.ndim - 2
    return _within_budget(
        int(_nd_workspace_bytes(_lib.get_lib(), nd, int(x.shape[0]), int(x.shape[1]),
                                _lib.i64_array([int(d) for d in x.shape[2:]]),
                                _lib.i64_array([int(d) for d in k.shape[1:]]), kbatch, periodic, _lib.NSQ_DIR_BWD)),
        x.device)


@custom_op("nsq_hip::fftconv_nd", mutates_args=())
def fftconv_nd_op(x: torch.Tensor, k: torch.Tensor, s: Optional[torch.Tensor], kbatch: int, periodic: int,
                  keep: bool) -> tuple[torch.Tensor, torch.Tensor]:
    """2D/3D non-causal FFT conv forward; x ``[B, H, *S]``, k ``[kbatch*H, *K]`` float32, s ``[H]`` or None,
    ``periodic`` bit d = axis d circular.  ``(y, state)`` as :func:`causal_fftconv1d_op`."""
    y = torch.empty_like(x)
    state = torch.empty(_nd_state_bytes(x, k, kbatch, periodic, keep), dtype=torch.uint8, device=x.device)
    fftconv_nd_fwd_raw(x, k, s, y, kbatch, state if keep and state.numel() else None, periodic)
    return y, state


@fftconv_nd_op.register_fake
def _(x, k, s, kbatch, periodic, keep):
    return torch.empty_like(x), x.new_empty(_nd_state_bytes(x, k, kbatch, periodic, keep), dtype=torch.uint8)


@custom_op("nsq_hip::fftconv_nd_backward", mutates_args=("state",))
def fftconv_nd_backward_op(g: torch.Tensor, x: torch.Tensor, k: torch.Tensor, s: Optional[torch.Tensor],
                           state: torch.Tensor, kbatch: int, periodic: int) -> tuple[torch.Tensor, torch.Tensor,
                                                                                     torch.Tensor]:
    """Gradients ``(gx, gk, gs)`` of :func:`fftconv_nd_op` (gs ``[kbatch*H]`` partials, empty without a shortcut)."""
    gx = torch.empty_like(x)
    gk = torch.empty_like(k)
    gs = torch.empty(kbatch * x.shape[1] if s is not None else 0, dtype=torch.float32, device=x.device)
    has = state.numel() > 0
    fftconv_nd_bwd_raw(g, x, k, s, gx, gk, gs if s is not None else None, kbatch, state if has else None,
                       fwd_state=has, periodic=periodic)
    return gx, gk, gs


@fftconv_nd_backward_op.register_fake
def _(g, x, k, s, state, kbatch, periodic):
    return torch.empty_like(x), torch.empty_like(k), x.new_empty(kbatch * x.shape[1] if s is not None else 0,
                                                                 dtype=torch.float32)


def _nd_setup(ctx, inputs, output):
    x, k, s, kbatch, periodic, _keep = inputs
    # the second output is internal (state kept for the backward): no gradient flows into it, and none is
    # materialized for it (autograd would otherwise fill a zero tensor of its size before every backward)
    ctx.mark_non_differentiable(output[1])
    ctx.set_materialize_grads(False)
    ctx.save_for_backward(x, k, s)
    ctx.state = output[1]
    ctx.kbatch, ctx.periodic = kbatch, periodic


def _nd_backward(ctx, gy, _gstate):
    x, k, s = ctx.saved_tensors
    state = _take_state(ctx)
    g = channels_first_contiguous(gy.to(x.dtype))
    gx, gk, gs = fftconv_nd_backward_op(g, x, k, s, state, ctx.kbatch, ctx.periodic)
    return gx, gk, _shortcut_grad(gs, s, ctx.kbatch, x.shape[1]), None, None, None


fftconv_nd_op.register_autograd(_nd_backward, setup_context=_nd_setup)


def _nd_core(x: torch.Tensor, kernel: torch.Tensor, shortcut: torch.Tensor | None, nd: int,
             periodic: int = 0) -> torch.Tensor:
    if x.ndim != nd + 2:
        raise ValueError(f"x must be [B, H, {', '.join('S%d' % i for i in range(nd))}]; got {tuple(x.shape)}")
    B, H = x.shape[:2]
    if kernel.ndim == nd + 1:
        kernel = kernel.unsqueeze(0)
    assert kernel.ndim == nd + 2, f"Unexpected kernel shape: {tuple(kernel.shape)}."
    assert kernel.shape[0] in (1, B), (
        f"Leading dimension must be 1 or batch_size ({B}). Got kernel.shape={tuple(kernel.shape)}."
    )
    assert kernel.shape[1] == H, "Input and kernel must have the same number of channels (H)."
    for d in range(nd):
        if (periodic >> d) & 1:
            assert kernel.shape[2 + d] <= x.shape[2 + d], (
                f"K must be <= N on periodic axis {d}: K={kernel.shape[2 + d]}, N={x.shape[2 + d]}."
            )
        else:
            assert kernel.shape[2 + d] <= 2 * x.shape[2 + d], (
                f"Kernel size must be less than 2 * S_{d}. Got {kernel.shape[2 + d]}."
            )
    kbatch = kernel.shape[0]
    input_dtype = x.dtype
    compute_dtype = input_dtype if input_dtype in _lib.NSQ_DTYPE else torch.float32
    xc = channels_first_contiguous(x.to(compute_dtype))
    kc = channels_first_contiguous(kernel.float()).reshape(kbatch * H, *kernel.shape[2:])
    sc = None
    if shortcut is not None:
        if shortcut.shape != (H,):
            raise ValueError(f"shortcut must have shape ({H},); got {tuple(shortcut.shape)}")
        sc = shortcut.to(input_dtype).to(compute_dtype).contiguous()
    y, _ = fftconv_nd_op(xc, kc, sc, kbatch, int(periodic), _grad_wanted(xc, kc, sc))
    return y.to(input_dtype)


def _chunked(fn, x, kernel, shortcut, chunk_size, nd):
    if chunk_size is None:
        chunk_size = _DEFAULT_CHUNK_SIZE
    H = x.shape[1]
    if H <= chunk_size:
        return fn(x, kernel, shortcut)
    k = kernel if kernel.ndim == nd + 2 else kernel.unsqueeze(0)
    outs = []
    for start in range(0, H, chunk_size):
        end = min(start + chunk_size, H)
        outs.append(fn(x[:, start:end], k[:, start:end], None if shortcut is None else shortcut[start:end]))
    return torch.cat(outs, dim=1)


# ---------------------------------------------------------------------------
# Non-causal 1D on the fused kernels: zero-padded "same" (periodic 0) or
# circular (periodic 1), both an output shift through the filter's ramp.
# ---------------------------------------------------------------------------
def mixed_fftconv1d_fwd_raw(x, k, s, y, kbatch: int, periodic: int):
    """Launch ``nsq_mixed_fftconv1d_fwd``: x/y ``[B, H, L]``, k float32 ``[kbatch*H, K]``, s ``[H]`` or None."""
    lib = _lib.get_lib()
    _lib.check_device(x)
    B, H, L = x.shape
    dt = _lib.dtype_code(x.dtype)
    ws = _workspace(x.device, lib.nsq_mixed_fftconv1d_workspace_bytes(B, H, L, k.shape[-1], kbatch, int(periodic),
                                                                       dt, _lib.NSQ_DIR_FWD))
    _lib.check(lib.nsq_mixed_fftconv1d_fwd(
        x.data_ptr(), k.data_ptr(), _lib.ptr(s), y.data_ptr(), dt, B, H, L, k.shape[-1], kbatch, int(periodic),
        _lib.ptr(ws), 0 if ws is None else ws.numel(), _lib.stream_ptr(x.device)))
    return y


def mixed_fftconv1d_bwd_raw(g, x, k, s, gx, gk, gs, kbatch: int, periodic: int):
    """Launch ``nsq_mixed_fftconv1d_bwd`` (gk ``[kbatch*H, K]``, gs ``[kbatch*H]`` partials or None)."""
    lib = _lib.get_lib()
    _lib.check_device(x)
    B, H, L = x.shape
    dt = _lib.dtype_code(x.dtype)
    ws = _workspace(x.device, lib.nsq_mixed_fftconv1d_workspace_bytes(B, H, L, k.shape[-1], kbatch, int(periodic),
                                                                       dt, _lib.NSQ_DIR_BWD))
    _lib.check(lib.nsq_mixed_fftconv1d_bwd(
        g.data_ptr(), x.data_ptr(), k.data_ptr(), _lib.ptr(s), gx.data_ptr(), gk.data_ptr(), _lib.ptr(gs), dt, B, H,
        L, k.shape[-1], kbatch, int(periodic), _lib.ptr(ws), 0 if ws is None else ws.numel(),
        _lib.stream_ptr(x.device)))


@custom_op("nsq_hip::shifted_fftconv1d", mutates_args=())
def shifted_fftconv1d_op(x: torch.Tensor, k: torch.Tensor, s: Optional[torch.Tensor], kbatch: int,
                         periodic: int) -> torch.Tensor:
    """Non-causal 1D FFT conv (periodic 1: circular; 0: zero-padded "same"); x ``[B, H, L]``, k ``[kbatch*H, K]``
    float32, s ``[H]`` or None."""
    y = torch.empty_like(x)
    mixed_fftconv1d_fwd_raw(x, k, s, y, kbatch, periodic)
    return y


@shifted_fftconv1d_op.register_fake
def _(x, k, s, kbatch, periodic):
    return torch.empty_like(x)


@custom_op("nsq_hip::shifted_fftconv1d_backward", mutates_args=())
def shifted_fftconv1d_backward_op(g: torch.Tensor, x: torch.Tensor, k: torch.Tensor, s: Optional[torch.Tensor],
                                  kbatch: int, periodic: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Gradients ``(gx, gk, gs)`` of :func:`shifted_fftconv1d_op` (gs partials, empty without a shortcut)."""
    gx = torch.empty_like(x)
    gk = torch.empty_like(k)
    gs = torch.empty(kbatch * x.shape[1] if s is not None else 0, dtype=torch.float32, device=x.device)
    mixed_fftconv1d_bwd_raw(g, x, k, s, gx, gk, gs if s is not None else None, kbatch, periodic)
    return gx, gk, gs


@shifted_fftconv1d_backward_op.register_fake
def _(g, x, k, s, kbatch, periodic):
    return torch.empty_like(x), torch.empty_like(k), x.new_empty(kbatch * x.shape[1] if s is not None else 0,
                                                                 dtype=torch.float32)


def _shifted_setup(ctx, inputs, output):
    x, k, s, kbatch, periodic = inputs
    ctx.save_for_backward(x, k, s)
    ctx.kbatch, ctx.periodic = kbatch, periodic


def _shifted_backward(ctx, gy):
    x, k, s = ctx.saved_tensors
    g = channels_first_contiguous(gy.to(x.dtype))
    gx, gk, gs = shifted_fftconv1d_backward_op(g, x, k, s, ctx.kbatch, ctx.periodic)
    return gx, gk, _shortcut_grad(gs, s, ctx.kbatch, x.shape[1]), None, None


shifted_fftconv1d_op.register_autograd(_shifted_backward, setup_context=_shifted_setup)


def shifted_fftconv1d(x: torch.Tensor, kernel: torch.Tensor, shortcut: torch.Tensor | None, periodic: int):
    """Cast and launch the 1D shifted conv (shapes already checked): kernel ``[1|B, H, K]``."""
    B, H, L = x.shape
    kbatch = kernel.shape[0]
    input_dtype = x.dtype
    compute_dtype = input_dtype if input_dtype in _lib.NSQ_DTYPE else torch.float32
    xc = channels_first_contiguous(x.to(compute_dtype))
    kc = channels_first_contiguous(kernel.float()).reshape(kbatch * H, kernel.shape[-1])
    sc = None if shortcut is None else shortcut.to(compute_dtype).contiguous()
    return shifted_fftconv1d_op(xc, kc, sc, kbatch, int(periodic)).to(input_dtype)


def fftconv1d_bhl(x: torch.Tensor, kernel: torch.Tensor, shortcut: torch.Tensor | None = None) -> torch.Tensor:
    """1D zero-padded non-causal ("same") FFT conv, BHL ``[B, H, L]`` (``fftconv.py:603-660``).

    ``y[n] = sum_j k[j] x[n + K//2 - j]`` with x zero outside ``[0, L)``, cast to
    ``x.dtype``, then ``+ shortcut * x``.  Kernel ``[1|B, H, K]``, ``K <= 2L``.
    Runs ``nsq_mixed_fftconv1d_*`` with ``periodic=0`` at FFT length
    ``pow2(L + ceil(K/2))`` (the reference's ``L + (K+1)//2`` gives the same
    result: every length from there on keeps the output window free of
    wrap-around): the fused kernels up to 16384, the 4-step plan up to 2^24;
    longer raises ``NotImplementedError``.
    """
    batch_size, hidden_dim, seq_len = x.shape
    assert len(kernel.shape) == 3, f"Unexpected kernel shape: {kernel.shape}."
    assert kernel.shape[0] in (1, batch_size), (
        f"Leading dimension must be 1 or batch_size ({batch_size}). Got kernel.shape={kernel.shape}."
    )
    kernel_len = kernel.shape[-1]
    assert kernel_len <= 2 * seq_len, f"Kernel length must be less than or equal to 2 * seq_len. Got {kernel_len}."
    if kernel.shape[1] != hidden_dim:
        raise ValueError(f"kernel has {kernel.shape[1]} channels, x has {hidden_dim}")
    if shortcut is not None:
        assert shortcut.dtype == x.dtype, f"shortcut.dtype ({shortcut.dtype}) must match x.dtype ({x.dtype})"
        assert shortcut.shape == (hidden_dim,)
    return shifted_fftconv1d(x, kernel, shortcut, 0)


def fftconv1d_bhl_w_reshape(x, kernel, shortcut=None):
    """BLH ``[B, L, H]`` input, kernel ``[1|B, K, H]`` (``fftconv.py:476-500``)."""
    y = fftconv1d_bhl(rearrange(x, "b l h -> b h l"), rearrange(kernel, "b l h -> b h l"), shortcut)
    return rearrange(y, "b h l -> b l h")


def fftconv1d_blh(x, kernel, shortcut=None):
    """Alias for :func:`fftconv1d_bhl_w_reshape` (``fftconv.py:235``)."""
    return fftconv1d_bhl_w_reshape(x, kernel, shortcut)


def fftconv1d_bhl_chunked(x, kernel, shortcut=None, chunk_size=None):
    """Channel-chunked zero-padded 1D (``fftconv_chunked.py:245-280``); bitwise equal to unchunked."""
    return _chunked(fftconv1d_bhl, x, kernel, shortcut, chunk_size, 1)


def fftconv1d_bhl_w_reshape_chunked(x, kernel, shortcut=None, chunk_size=None):
    """Chunked BLH zero-padded 1D."""
    y = fftconv1d_bhl_chunked(rearrange(x, "b l h -> b h l"), rearrange(kernel, "b l h -> b h l"), shortcut,
                              chunk_size)
    return rearrange(y, "b h l -> b l h")


def fftconv1d_blh_chunked(x, kernel, shortcut=None, chunk_size=None):
    """Alias for :func:`fftconv1d_bhl_w_reshape_chunked`."""
    return fftconv1d_bhl_w_reshape_chunked(x, kernel, shortcut, chunk_size)


def fftconv2d_bhl(x: torch.Tensor, kernel: torch.Tensor, shortcut: torch.Tensor | None = None) -> torch.Tensor:
    """2D zero-padded FFT conv, BHL ``[B, H, X, Y]`` (``fftconv_custom.py:133-160``).

    Kernel ``[1|B, H, Kx, Ky]`` or ``[H, Kx, Ky]`` (per-sample FiLM kernels are
    supported as in ``_subq_conv2d_bhl``, ``fftconv_custom.py:117-125``).
    Numerically matches ``nvsubquadratic.ops.fftconv.fftconv2d_fp32_bhl``
    (``fftconv.py:662-733``).
    """
    return _nd_core(x, kernel, shortcut, 2)


def fftconv2d_bhl_w_reshape(x, kernel, shortcut=None):
    """BLH ``[B, X, Y, H]`` input, kernel ``[1|B, Kx, Ky, H]`` (``fftconv_custom.py:163-175``)."""
    y = fftconv2d_bhl(rearrange(x, "b x y h -> b h x y"), rearrange(kernel, "b x y h -> b h x y"), shortcut)
    return rearrange(y, "b h x y -> b x y h")


def fftconv2d_blh(x, kernel, shortcut=None):
    """Alias for :func:`fftconv2d_bhl_w_reshape` (``fftconv_custom.py:178-184``)."""
    return fftconv2d_bhl_w_reshape(x, kernel, shortcut)


def fftconv2d_bhl_chunked(x, kernel, shortcut=None, chunk_size=None):
    """Channel-chunked 2D (``fftconv_custom.py:194-234``); bitwise equal to unchunked."""
    return _chunked(fftconv2d_bhl, x, kernel, shortcut, chunk_size, 2)


def fftconv2d_bhl_w_reshape_chunked(x, kernel, shortcut=None, chunk_size=None):
    """Chunked BLH 2D (``fftconv_custom.py:237-250``)."""
    y = fftconv2d_bhl_chunked(rearrange(x, "b x y h -> b h x y"), rearrange(kernel, "b x y h -> b h x y"),
                              shortcut, chunk_size)
    return rearrange(y, "b h x y -> b x y h")


def fftconv2d_blh_chunked(x, kernel, shortcut=None, chunk_size=None):
    """Alias for :func:`fftconv2d_bhl_w_reshape_chunked` (``fftconv_custom.py:253-260``)."""
    return fftconv2d_bhl_w_reshape_chunked(x, kernel, shortcut, chunk_size)


def fftconv3d_bhl(x: torch.Tensor, kernel: torch.Tensor, shortcut: torch.Tensor | None = None) -> torch.Tensor:
    """3D zero-padded FFT conv, BHL ``[B, H, X, Y, Z]``.

    Numerically matches ``nvsubquadratic.ops.fftconv.fftconv3d_fp32_bhl``
    (``fftconv.py:736-812``); the reference has no accelerated 3D kernel.
    """
    return _nd_core(x, kernel, shortcut, 3)


def fftconv3d_bhl_w_reshape(x, kernel, shortcut=None):
    """BLH ``[B, X, Y, Z, H]`` input (mirrors ``fftconv.py:522-538``)."""
    y = fftconv3d_bhl(rearrange(x, "b x y z h -> b h x y z"), rearrange(kernel, "b x y z h -> b h x y z"), shortcut)
    return rearrange(y, "b h x y z -> b x y z h")


def fftconv3d_blh(x, kernel, shortcut=None):
    """Alias for :func:`fftconv3d_bhl_w_reshape`."""
    return fftconv3d_bhl_w_reshape(x, kernel, shortcut)


def fftconv3d_bhl_chunked(x, kernel, shortcut=None, chunk_size=None):
    """Channel-chunked 3D (``fftconv_chunked.py`` semantics); bitwise equal to unchunked."""
    return _chunked(fftconv3d_bhl, x, kernel, shortcut, chunk_size, 3)


def fftconv3d_bhl_w_reshape_chunked(x, kernel, shortcut=None, chunk_size=None):
    """Chunked BLH 3D."""
    y = fftconv3d_bhl_chunked(rearrange(x, "b x y z h -> b h x y z"), rearrange(kernel, "b x y z h -> b h x y z"),
                              shortcut, chunk_size)
    return rearrange(y, "b h x y z -> b x y z h")


def fftconv3d_blh_chunked(x, kernel, shortcut=None, chunk_size=None):
    """Alias for :func:`fftconv3d_bhl_w_reshape_chunked`."""
    return fftconv3d_bhl_w_reshape_chunked(x, kernel, shortcut, chunk_size)
