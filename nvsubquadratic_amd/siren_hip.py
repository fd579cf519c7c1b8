r"""HIP implicit filter generation: the SIREN MLP of ``SIRENKernelND`` on the matrix cores.

Reference: ``nvsubquadratic/modules/kernels_nd.py`` -- ``SIRENPositionalEmbeddingND`` (:660-860) and
``SIRENKernelND`` (:876-1190): for the grid coordinates ``x`` (per axis ``2 * seq_len - 1`` points on
``[-1, 1]`` at the cache's step),

    a_0 = sin(W_0 x + b_0),   a_i = sin(W_i a_{i-1} + b_i),   k = W_out a_nh + b_out,

returned as ``[1, *grid, out_dim]``; ``CKConvND`` then crops it (causal: the second half,
``ckconv_nd.py:1149-1164``) and moves the channels first for the FFT conv.

How: ``nsq_siren_mlp_fwd`` evaluates the embedding and every hidden layer for 16 grid points per wave
on the matrix cores and writes only ``[a_nh^T; 1]`` (``[HD + 1, G]``) -- no per-layer activation reaches
HBM.  The readout (``nsq_siren_readout_fwd``: one point per lane, the W_out rows wave-uniform) writes the
filter straight as ``[out_dim, G]`` -- the layout the FFT convs read -- so neither the ``[G, out_dim]``
result nor its transpose exists; ``forward`` hands the reference's
``[1, *grid, out_dim]`` shape back as a view of it.  The readout's gradients come from one pass over the
filter gradient (``nsq_siren_readout_bwd``); the MLP backward (``nsq_siren_mlp_bwd``) recomputes the layers from the grid and reduces
every hidden weight gradient over the points in a fixed order.  fp32 throughout, as the reference
computes.

FiLM conditioning (``film_cfg``, ``kernels_nd.py:1165-1187``): :class:`KernelFiLMGenerator` maps the conditioning
vector to one ``(gamma, beta)`` pair per modulated layer (``modules/film.py:75``, a small torch MLP over ``[B,
cond_dim]``); the per-point work -- ``h = gamma * sin(z) + beta`` inside the hidden stack, the per-sample readout and
their gradients, ``gamma`` / ``beta`` gradients included -- runs in ``nsq_siren_mlp_film_{fwd,bwd}`` /
``nsq_siren_film_readout_fwd``, the filter coming out per sample, ``[B, out_dim, *grid]``.  Not covered: hidden and
embedding widths other than 16, 32, 64 or 128 (raised by the library).
"""

from __future__ import annotations

import math
from collections.abc import Sequence
from typing import Optional

import torch
from torch.library import custom_op

from . import _lib

__all__ = ["HipSIRENKernelND", "KernelFiLMGenerator", "siren_causal_fftconv1d", "siren_film_filter", "siren_filter",
           "siren_filter_op", "siren_grid"]


def _opt(t: Optional[torch.Tensor]) -> int | None:
    return None if t is None or t.numel() == 0 else t.data_ptr()


def _has(t: Optional[torch.Tensor]) -> bool:
    return t is not None and t.numel() > 0


def _mlp_fwd(grid: torch.Tensor, w0: torch.Tensor, b0: Optional[torch.Tensor], wh: torch.Tensor,
             bh: Optional[torch.Tensor], nh: int, HD: int) -> torch.Tensor:
    """``[a_nh^T; 1]`` ``[HD + 1, G]`` float32 for grid ``[G, d]`` (``nsq_siren_mlp_fwd``)."""
    lib = _lib.get_lib()
    _lib.check_device(grid)
    G, d = grid.shape
    act = torch.empty(HD + 1, G, dtype=torch.float32, device=grid.device)
    _lib.check(lib.nsq_siren_mlp_fwd(grid.data_ptr(), G, d, w0.data_ptr(), _opt(b0), w0.shape[0], wh.data_ptr(),
                                     _opt(bh), nh, HD, act.data_ptr(), G, _lib.stream_ptr(grid.device)))
    return act


# Split of the points for the readout's weight gradient: gk [H, G] x act^T [G, HD + 1] is a long-K product
# (K = G) that a single library GEMM runs at ~2 TB/s on MI355X; 16 batched slices of G / 16 points, summed
# in a fixed order, read gk at ~5 TB/s.
_GRAM_SPLIT = 16
_GRAM_SPLIT_MIN_G = 1 << 16


def _readout_gram(gk: torch.Tensor, rows: torch.Tensor) -> torch.Tensor:
    """``gk @ rows^T`` (``[H, K]``) for ``gk [H, G]``, ``rows [K, G]``, both with unit column stride."""
    H, G = gk.shape
    K = rows.shape[0]
    if G < _GRAM_SPLIT_MIN_G:
        return torch.mm(gk, rows.t())
    c = _GRAM_SPLIT
    m = G // c
    n = c * m
    part = torch.bmm(rows[:, :n].view(K, c, m).transpose(0, 1), gk[:, :n].view(H, c, m).permute(1, 2, 0))
    out = part.sum(0)  # [K, H]
    if n < G:
        out = out + torch.mm(rows[:, n:], gk[:, n:].t())
    return out.t()


def _readout_backward(gk: torch.Tensor, act: torch.Tensor, wout: torch.Tensor,
                      has_bout: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``(gact [HD, G], gwout [H, HD], gbout [H] or empty)`` for ``gk [H, G]`` (unit column stride).

    ``nsq_siren_readout_bwd`` reads gk once (bf16-split matrix products, fp32 accumulation); at HD = 128, which
    that kernel does not take, two library GEMMs (``K = H``, and ``K = G`` in fixed-order slices)."""
    lib = _lib.get_lib()
    H, HD = wout.shape
    G = gk.shape[1]
    dev = gk.device
    need = lib.nsq_siren_readout_bwd_workspace_bytes(H, HD, G, 1)
    if need == 0:
        gact = torch.mm(gk.t(), wout).t()  # [HD, G] view of [G, HD]
        gw_ext = _readout_gram(gk, act if has_bout else act[:HD])  # [H, HD (+1)]
        return gact, gw_ext[:, :HD].contiguous(), (gw_ext[:, HD].contiguous() if has_bout else wout.new_empty(0))
    gact = torch.empty(HD, G, dtype=torch.float32, device=dev)
    gwout = torch.empty(H, HD, dtype=torch.float32, device=dev)
    gbout = torch.empty(H if has_bout else 0, dtype=torch.float32, device=dev)
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    _lib.check(lib.nsq_siren_readout_bwd(gk.data_ptr(), gk.stride(0), act.data_ptr(), act.stride(0), wout.data_ptr(),
                                         H, HD, G, 1, gact.data_ptr(), gwout.data_ptr(), _opt(gbout), ws.data_ptr(),
                                         ws.numel(), _lib.stream_ptr(dev)))
    return gact, gwout, gbout


@custom_op("nsq_hip::siren_filter", mutates_args=())
def siren_filter_op(grid: torch.Tensor, w0: torch.Tensor, b0: Optional[torch.Tensor], wh: torch.Tensor,
                    bh: Optional[torch.Tensor], wout: torch.Tensor, bout: Optional[torch.Tensor],
                    nh: int) -> tuple[torch.Tensor, torch.Tensor]:
    """``(k [H, G], act [HD + 1, G])`` float32 for grid ``[G, d]``: the embedding ``w0 [E, d]``, ``b0``,
    ``nh`` hidden layers packed back to back in ``wh`` (biases in ``bh``) and the readout ``wout [H, HD]``,
    ``bout``.  ``act = [a_nh^T; 1]`` is the forward state the backward reads."""
    HD = wout.shape[1]
    H, G = wout.shape[0], grid.shape[0]
    act = _mlp_fwd(grid, w0, b0, wh, bh, nh, HD)
    k = torch.empty(H, G, dtype=torch.float32, device=grid.device)
    _lib.check(_lib.get_lib().nsq_siren_readout_fwd(wout.data_ptr(), _opt(bout), H, HD, act.data_ptr(), act.stride(0),
                                                    G, k.data_ptr(), _lib.stream_ptr(grid.device)))
    return k, act


@siren_filter_op.register_fake
def _(grid, w0, b0, wh, bh, wout, bout, nh):
    G = grid.shape[0]
    return grid.new_empty(wout.shape[0], G), grid.new_empty(wout.shape[1] + 1, G)


@custom_op("nsq_hip::siren_filter_backward", mutates_args=())
def siren_filter_backward_op(gk: torch.Tensor, act: torch.Tensor, grid: torch.Tensor, w0: torch.Tensor,
                             b0: Optional[torch.Tensor], wh: torch.Tensor, bh: Optional[torch.Tensor],
                             wout: torch.Tensor, nh: int, has_bout: bool) -> tuple[torch.Tensor, torch.Tensor,
                                                                                   torch.Tensor, torch.Tensor,
                                                                                   torch.Tensor, torch.Tensor]:
    """Gradients ``(gw0, gb0, gwh, gbh, gwout, gbout)`` for ``gk [H, G]`` (empty where a bias is absent): the
    readout's gradients in one pass over gk (``nsq_siren_readout_bwd``), then ``nsq_siren_mlp_bwd`` on
    ``gact = wout^T gk`` ``[HD, G]``."""
    if gk.stride(1) != 1:
        gk = gk.contiguous()
    gact, gwout, gbout = _readout_backward(gk, act, wout, has_bout)
    return (*_mlp_backward(gact, grid, w0, b0, wh, bh, nh, wout.shape[1]), gwout, gbout)


def _mlp_backward(gact: torch.Tensor, grid: torch.Tensor, w0: torch.Tensor, b0: Optional[torch.Tensor],
                  wh: torch.Tensor, bh: Optional[torch.Tensor], nh: int,
                  HD: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """``(gw0, gb0, gwh, gbh)`` of the hidden stack for ``gact [HD, G]`` (any strides; rows >= HD are not read):
    ``nsq_siren_mlp_bwd`` recomputes the layers from the grid."""
    lib = _lib.get_lib()
    G, d = grid.shape
    E = w0.shape[0]
    dev = grid.device
    gw0, gwh = torch.empty_like(w0), torch.empty_like(wh)
    gb0 = torch.empty(E if _has(b0) else 0, device=dev)
    gbh = torch.empty(nh * HD if _has(bh) else 0, device=dev)
    need = lib.nsq_siren_mlp_bwd_workspace_bytes(G, d, E, nh, HD)
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    _lib.check(lib.nsq_siren_mlp_bwd(gact.data_ptr(), gact.stride(0), gact.stride(1), grid.data_ptr(), G, d,
                                     w0.data_ptr(), _opt(b0), E, wh.data_ptr(), _opt(bh), nh, HD, gw0.data_ptr(),
                                     _opt(gb0), gwh.data_ptr(), _opt(gbh), ws.data_ptr(), ws.numel(),
                                     _lib.stream_ptr(dev)))
    return gw0, gb0, gwh, gbh


@siren_filter_backward_op.register_fake
def _(gk, act, grid, w0, b0, wh, bh, wout, nh, has_bout):
    HD = wout.shape[1]
    return (torch.empty_like(w0), w0.new_empty(w0.shape[0] if _has(b0) else 0), torch.empty_like(wh),
            wh.new_empty(nh * HD if _has(bh) else 0), torch.empty_like(wout),
            wout.new_empty(wout.shape[0] if has_bout else 0))


def _setup(ctx, inputs, output):
    grid, w0, b0, wh, bh, wout, bout, nh = inputs
    ctx.mark_non_differentiable(output[1])
    ctx.set_materialize_grads(False)
    ctx.save_for_backward(grid, w0, b0, wh, bh, wout, output[1])
    ctx.nh = nh
    ctx.has_bout = bout is not None


def _backward(ctx, gk, _gact):
    grid, w0, b0, wh, bh, wout, act = ctx.saved_tensors
    if gk is None:
        return (None,) * 8
    gw0, gb0, gwh, gbh, gwout, gbout = siren_filter_backward_op(gk.float(), act, grid, w0, b0, wh, bh, wout, ctx.nh,
                                                                ctx.has_bout)
    return (None, gw0, gb0 if b0 is not None else None, gwh, gbh if bh is not None else None, gwout,
            gbout if ctx.has_bout else None, None)


siren_filter_op.register_autograd(_backward, setup_context=_setup)


def _readout_backward_samples(gk: torch.Tensor, act: torch.Tensor, wout: torch.Tensor,
                              has_bout: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """:func:`_readout_backward` for per-sample filters ``gk [nb, H, G]``, ``act [nb, HD + 1, G]``: ``gact [nb, HD,
    G]`` per sample, ``gwout`` / ``gbout`` summed over the samples."""
    lib = _lib.get_lib()
    nb, H, G = gk.shape
    HD = wout.shape[1]
    dev = gk.device
    need = lib.nsq_siren_readout_bwd_workspace_bytes(H, HD, G, nb)
    if need == 0:  # HD = 128: library products in float32
        gact = torch.matmul(wout.t().contiguous(), gk)
        gw_ext = torch.matmul(gk.transpose(0, 1).reshape(H, nb * G),
                              (act if has_bout else act[:, :HD]).transpose(0, 1).reshape(-1, nb * G).t())
        return gact, gw_ext[:, :HD].contiguous(), (gw_ext[:, HD].contiguous() if has_bout else wout.new_empty(0))
    gact = torch.empty(nb, HD, G, dtype=torch.float32, device=dev)
    gwout = torch.empty(H, HD, dtype=torch.float32, device=dev)
    gbout = torch.empty(H if has_bout else 0, dtype=torch.float32, device=dev)
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    _lib.check(lib.nsq_siren_readout_bwd(gk.data_ptr(), gk.stride(1), act.data_ptr(), act.stride(1), wout.data_ptr(),
                                         H, HD, G, nb, gact.data_ptr(), gwout.data_ptr(), _opt(gbout), ws.data_ptr(),
                                         ws.numel(), _lib.stream_ptr(dev)))
    return gact, gwout, gbout


@custom_op("nsq_hip::siren_film_filter", mutates_args=())
def siren_film_filter_op(grid: torch.Tensor, w0: torch.Tensor, b0: Optional[torch.Tensor], wh: torch.Tensor,
                         bh: Optional[torch.Tensor], wout: torch.Tensor, bout: Optional[torch.Tensor], film: torch.Tensor,
                         nh: int, film_first: bool) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-sample filters ``(k [nb, H, G], act [nb, HD + 1, G])`` for FiLM parameters ``film [nb, nfilm, 2, HD]``
    (``nsq_siren_mlp_film_fwd``, ``nsq_siren_film_readout_fwd``)."""
    lib = _lib.get_lib()
    _lib.check_device(grid)
    G, d = grid.shape
    H, HD = wout.shape
    nb = film.shape[0]
    act = torch.empty(nb, HD + 1, G, dtype=torch.float32, device=grid.device)
    st = _lib.stream_ptr(grid.device)
    _lib.check(lib.nsq_siren_mlp_film_fwd(grid.data_ptr(), G, d, w0.data_ptr(), _opt(b0), w0.shape[0], wh.data_ptr(),
                                          _opt(bh), nh, HD, film.data_ptr(), nb, int(film_first), act.data_ptr(), G,
                                          st))
    k = torch.empty(nb, H, G, dtype=torch.float32, device=grid.device)
    _lib.check(lib.nsq_siren_film_readout_fwd(wout.data_ptr(), _opt(bout), H, HD, act.data_ptr(), G, G, nb,
                                              k.data_ptr(), st))
    return k, act


@siren_film_filter_op.register_fake
def _(grid, w0, b0, wh, bh, wout, bout, film, nh, film_first):
    G, nb = grid.shape[0], film.shape[0]
    return grid.new_empty(nb, wout.shape[0], G), grid.new_empty(nb, wout.shape[1] + 1, G)


@custom_op("nsq_hip::siren_film_filter_backward", mutates_args=())
def siren_film_filter_backward_op(gk: torch.Tensor, act: torch.Tensor, grid: torch.Tensor, w0: torch.Tensor,
                                  b0: Optional[torch.Tensor], wh: torch.Tensor, bh: Optional[torch.Tensor],
                                  wout: torch.Tensor, film: torch.Tensor, nh: int, film_first: bool,
                                  has_bout: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
                                                           torch.Tensor, torch.Tensor, torch.Tensor]:
    """Gradients ``(gw0, gb0, gwh, gbh, gwout, gbout, gfilm)`` of the per-sample filters (weights summed over the
    samples, ``gfilm [nb, nfilm, 2, HD]`` per sample)."""
    lib = _lib.get_lib()
    G, d = grid.shape
    H, HD = wout.shape
    E = w0.shape[0]
    nb = film.shape[0]
    dev = grid.device
    gk = gk.contiguous()
    gact, gwout, gbout = _readout_backward_samples(gk, act, wout, has_bout)
    gw0, gwh = torch.empty_like(w0), torch.empty_like(wh)
    gb0 = torch.empty(E if _has(b0) else 0, device=dev)
    gbh = torch.empty(nh * HD if _has(bh) else 0, device=dev)
    gfilm = torch.empty_like(film)
    need = lib.nsq_siren_mlp_film_bwd_workspace_bytes(G, d, E, nh, HD, nb, int(film_first))
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    _lib.check(lib.nsq_siren_mlp_film_bwd(gact.data_ptr(), gact.stride(1), gact.stride(2), gact.stride(0),
                                          grid.data_ptr(), G, d, w0.data_ptr(), _opt(b0), E, wh.data_ptr(), _opt(bh),
                                          nh, HD, film.data_ptr(), nb, int(film_first), gw0.data_ptr(), _opt(gb0),
                                          gwh.data_ptr(), _opt(gbh), gfilm.data_ptr(), ws.data_ptr(), ws.numel(),
                                          _lib.stream_ptr(dev)))
    return gw0, gb0, gwh, gbh, gwout, gbout, gfilm


@siren_film_filter_backward_op.register_fake
def _(gk, act, grid, w0, b0, wh, bh, wout, film, nh, film_first, has_bout):
    HD = wout.shape[1]
    return (torch.empty_like(w0), w0.new_empty(w0.shape[0] if _has(b0) else 0), torch.empty_like(wh),
            wh.new_empty(nh * HD if _has(bh) else 0), torch.empty_like(wout),
            wout.new_empty(wout.shape[0] if has_bout else 0), torch.empty_like(film))


def _film_setup(ctx, inputs, output):
    grid, w0, b0, wh, bh, wout, bout, film, nh, film_first = inputs
    ctx.mark_non_differentiable(output[1])
    ctx.set_materialize_grads(False)
    ctx.save_for_backward(grid, w0, b0, wh, bh, wout, film, output[1])
    ctx.nh, ctx.film_first = nh, film_first
    ctx.has_bout = bout is not None


def _film_backward(ctx, gk, _gact):
    grid, w0, b0, wh, bh, wout, film, act = ctx.saved_tensors
    if gk is None:
        return (None,) * 10
    gw0, gb0, gwh, gbh, gwout, gbout, gfilm = siren_film_filter_backward_op(
        gk.float(), act, grid, w0, b0, wh, bh, wout, film, ctx.nh, ctx.film_first, ctx.has_bout)
    return (None, gw0, gb0 if b0 is not None else None, gwh, gbh if bh is not None else None, gwout,
            gbout if ctx.has_bout else None, gfilm, None, None)


siren_film_filter_op.register_autograd(_film_backward, setup_context=_film_setup)


def siren_film_filter(grid: torch.Tensor, w0: torch.Tensor, b0: torch.Tensor | None,
                      hidden_w: Sequence[torch.Tensor], hidden_b: Sequence[torch.Tensor] | None, wout: torch.Tensor,
                      bout: torch.Tensor | None, film_params: Sequence[tuple[torch.Tensor, torch.Tensor]],
                      film_first: bool = False) -> torch.Tensor:
    """Functional FiLM form: per-sample filters ``[B, H, G]`` for the ``(gamma, beta)`` pairs ``film_params`` (each
    ``[B, HD]``, in :class:`KernelFiLMGenerator`'s order: with ``film_first`` the first pair modulates the positional
    embedding, the rest the hidden layers in order)."""
    f = lambda t: None if t is None else t.float().contiguous()  # noqa: E731
    wh = torch.cat([w.float().reshape(-1) for w in hidden_w])
    bh = None if hidden_b is None else torch.cat([b.float().reshape(-1) for b in hidden_b])
    film = torch.stack([torch.stack([g.float(), b.float()], dim=1) for g, b in film_params], dim=1).contiguous()
    return siren_film_filter_op(f(grid), f(w0), f(b0), wh, bh, f(wout), f(bout), film, len(hidden_w),
                                bool(film_first))[0]


def siren_filter(grid: torch.Tensor, w0: torch.Tensor, b0: torch.Tensor | None, hidden_w: Sequence[torch.Tensor],
                 hidden_b: Sequence[torch.Tensor] | None, wout: torch.Tensor, bout: torch.Tensor | None) -> torch.Tensor:
    """Functional form: filter ``[H, G]`` (float32) at the ``G`` points of ``grid [G, d]``.

    ``hidden_w[i]`` is the weight of hidden linear ``i`` (``[HD, E]`` then ``[HD, HD]``), ``hidden_b``
    their biases (None: no biases); every weight is read as float32, as the reference computes.  The
    hidden stack runs in ``nsq_siren_mlp_fwd``, the readout in ``nsq_siren_readout_fwd``; the readout's
    gradients come from one pass over the filter gradient (``nsq_siren_readout_bwd``)."""
    f = lambda t: None if t is None else t.float().contiguous()  # noqa: E731
    wh = torch.cat([w.float().reshape(-1) for w in hidden_w])
    bh = None if hidden_b is None else torch.cat([b.float().reshape(-1) for b in hidden_b])
    return siren_filter_op(f(grid), f(w0), f(b0), wh, bh, f(wout), f(bout), len(hidden_w))[0]


# ---------------------------------------------------------------------------
# Causal 1D conv with the SIREN filter kept out of HBM (nsq_siren_fftconv1d_causal_*): CKConvND's causal path
# (ckconv_nd.py:1149-1164, the generator's filter cropped to its causal half, then fftconv.py:546-600) as the
# hidden stack, then one conv op that forms the filter's column transforms from the transformed activations
# and returns the readout's gradients from the filter gradient's spectrum.
# ---------------------------------------------------------------------------
@custom_op("nsq_hip::siren_mlp", mutates_args=())
def siren_mlp_op(grid: torch.Tensor, w0: torch.Tensor, b0: Optional[torch.Tensor], wh: torch.Tensor,
                 bh: Optional[torch.Tensor], nh: int, HD: int) -> torch.Tensor:
    """``[a_nh^T; 1]`` ``[HD + 1, G]`` float32: the hidden stack's output with the ones row (the readout's
    input, bias included)."""
    return _mlp_fwd(grid, w0, b0, wh, bh, nh, HD)


@siren_mlp_op.register_fake
def _(grid, w0, b0, wh, bh, nh, HD):
    return grid.new_empty(HD + 1, grid.shape[0])


@custom_op("nsq_hip::siren_mlp_backward", mutates_args=())
def siren_mlp_backward_op(gact: torch.Tensor, grid: torch.Tensor, w0: torch.Tensor, b0: Optional[torch.Tensor],
                          wh: torch.Tensor, bh: Optional[torch.Tensor], nh: int,
                          HD: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """``(gw0, gb0, gwh, gbh)`` for ``gact [HD + 1, G]`` (the ones row's gradient is ignored)."""
    return _mlp_backward(gact, grid, w0, b0, wh, bh, nh, HD)


@siren_mlp_backward_op.register_fake
def _(gact, grid, w0, b0, wh, bh, nh, HD):
    return (torch.empty_like(w0), w0.new_empty(w0.shape[0] if _has(b0) else 0), torch.empty_like(wh),
            wh.new_empty(nh * HD if _has(bh) else 0))


def _mlp_setup(ctx, inputs, output):
    grid, w0, b0, wh, bh, nh, HD = inputs
    ctx.save_for_backward(grid, w0, b0, wh, bh)
    ctx.meta = (nh, HD)


def _mlp_backward_fn(ctx, gact):
    grid, w0, b0, wh, bh = ctx.saved_tensors
    nh, HD = ctx.meta
    gw0, gb0, gwh, gbh = siren_mlp_backward_op(gact.float(), grid, w0, b0, wh, bh, nh, HD)
    return None, gw0, gb0 if b0 is not None else None, gwh, gbh if bh is not None else None, None, None


siren_mlp_op.register_autograd(_mlp_backward_fn, setup_context=_mlp_setup)


def _siren_conv_ws_bytes(B: int, H: int, L: int, K: int, HD: int) -> int:
    return int(_lib.get_lib().nsq_siren_fftconv1d_causal_workspace_bytes(B, H, L, K, HD))


@custom_op("nsq_hip::siren_readout_causal_fftconv1d", mutates_args=())
def siren_readout_causal_fftconv1d_op(x: torch.Tensor, act: torch.Tensor, wout: torch.Tensor,
                                      bout: Optional[torch.Tensor], s: Optional[torch.Tensor],
                                      keep: bool) -> tuple[torch.Tensor, torch.Tensor]:
    """Causal conv of ``x [B, H, L]`` (contiguous) with the filter ``k = wout @ act[:HD] + bout`` (``act [HD + 1,
    K]``, last row ones), which is never formed.  Returns ``(y, state)``: with ``keep`` the workspace, in which
    the forward leaves the transformed x, filter and activations for the backward, else empty."""
    lib = _lib.get_lib()
    _lib.check_device(x)
    B, H, L = x.shape
    HD, K = wout.shape[1], act.shape[1]
    y = torch.empty_like(x)
    ws = torch.empty(_siren_conv_ws_bytes(B, H, L, K, HD), dtype=torch.uint8, device=x.device)
    _lib.check(lib.nsq_siren_fftconv1d_causal_fwd(x.data_ptr(), act.data_ptr(), act.stride(0), wout.data_ptr(),
                                                  _opt(bout), HD, _opt(s), y.data_ptr(), _lib.dtype_code(x.dtype), B,
                                                  H, L, K, ws.data_ptr(), ws.numel(), _lib.stream_ptr(x.device)))
    return y, (ws if keep else ws.new_empty(0))


@siren_readout_causal_fftconv1d_op.register_fake
def _(x, act, wout, bout, s, keep):
    B, H, L = x.shape
    n = _siren_conv_ws_bytes(B, H, L, act.shape[1], wout.shape[1]) if keep else 0
    return torch.empty_like(x), x.new_empty(n, dtype=torch.uint8)


@custom_op("nsq_hip::siren_readout_causal_fftconv1d_backward", mutates_args=("state",))
def siren_readout_causal_fftconv1d_backward_op(
        g: torch.Tensor, x: torch.Tensor, act: torch.Tensor, wout: torch.Tensor, bout: Optional[torch.Tensor],
        s: Optional[torch.Tensor], state: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor,
                                                                 torch.Tensor, torch.Tensor]:
    """``(gx, gact [HD + 1, K] (ones row zero), gwout, gbout, gs)``, gbout / gs empty without bout / s; a non-empty
    ``state`` is the forward's workspace and is consumed (overwritten)."""
    lib = _lib.get_lib()
    B, H, L = x.shape
    HD, K = wout.shape[1], act.shape[1]
    dev = x.device
    has = state.numel() > 0
    ws = state if has else torch.empty(_siren_conv_ws_bytes(B, H, L, K, HD), dtype=torch.uint8, device=dev)
    gx = torch.empty_like(x)
    gact = torch.empty(HD + 1, K, dtype=torch.float32, device=dev)
    gact[HD].zero_()
    gwout = torch.empty_like(wout)
    gbout = torch.empty(H if bout is not None else 0, dtype=torch.float32, device=dev)
    gs = torch.empty(H if s is not None else 0, dtype=torch.float32, device=dev)
    _lib.check(lib.nsq_siren_fftconv1d_causal_bwd(
        g.data_ptr(), x.data_ptr(), act.data_ptr(), act.stride(0), wout.data_ptr(), _opt(bout), HD, _opt(s),
        gx.data_ptr(), gact.data_ptr(), gwout.data_ptr(), _opt(gbout), _opt(gs), _lib.dtype_code(x.dtype), B, H, L,
        K, ws.data_ptr(), ws.numel(), int(has), _lib.stream_ptr(dev)))
    return gx, gact, gwout, gbout, gs


@siren_readout_causal_fftconv1d_backward_op.register_fake
def _(g, x, act, wout, bout, s, state):
    H = x.shape[1]
    return (torch.empty_like(x), act.new_empty(act.shape), torch.empty_like(wout),
            wout.new_empty(H if bout is not None else 0), wout.new_empty(H if s is not None else 0))


def _sconv_setup(ctx, inputs, output):
    x, act, wout, bout, s, _keep = inputs
    ctx.mark_non_differentiable(output[1])
    ctx.set_materialize_grads(False)
    ctx.save_for_backward(x, act, wout, bout, s)
    ctx.state = output[1]  # consumed in place by the backward: kept on ctx, not saved (version checks)


def _sconv_backward(ctx, gy, _gstate):
    x, act, wout, bout, s = ctx.saved_tensors
    if gy is None:
        return (None,) * 6
    state = ctx.state
    ctx.state = state.new_empty(0)  # a second backward (retain_graph) recomputes the transforms
    gx, gact, gwout, gbout, gs = siren_readout_causal_fftconv1d_backward_op(gy.to(x.dtype).contiguous(), x, act, wout,
                                                                            bout, s, state)
    return (gx, gact, gwout, gbout if bout is not None else None, gs.to(s.dtype) if s is not None else None, None)


siren_readout_causal_fftconv1d_op.register_autograd(_sconv_backward, setup_context=_sconv_setup)


def siren_conv_fits(B: int, H: int, L: int, K: int, HD: int) -> bool:
    """Whether ``nsq_siren_fftconv1d_causal_*`` takes the shape: the 4-step plan (FFT lengths 2^15 .. 2^23,
    ``K <= L + 1``) with ``HD`` in {16, 32, 64}.  Shorter convs run the fused plan, which reads the filter."""
    return _siren_conv_ws_bytes(B, H, L, K, HD) > 0


def siren_causal_fftconv1d(x: torch.Tensor, grid: torch.Tensor, w0: torch.Tensor, b0: torch.Tensor | None,
                           hidden_w: Sequence[torch.Tensor], hidden_b: Sequence[torch.Tensor] | None,
                           wout: torch.Tensor, bout: torch.Tensor | None,
                           shortcut: torch.Tensor | None = None) -> torch.Tensor:
    """Causal 1D FFT conv of ``x [B, H, L]`` with the SIREN filter at the ``K`` points of ``grid [K, 1]``:
    ``causal_fftconv1d_bhl(x, siren_filter(grid, ...), shortcut)`` with the same arguments, computed without the
    filter ``[H, K]`` or its gradient in HBM where :func:`siren_conv_fits` (else exactly that composition).

    The forward transforms the HD + 1 activation rows once and forms each channel's filter transform as
    ``sum_j wout[h, j] C(a_j) + bout[h] C(1)`` (the column pass C is linear); the backward reads the filter
    gradient's spectrum once for the readout's gradients (the inverse column pass's adjoint is C / N) and
    inverse-transforms only the HD rows of ``wout^T`` times it.  fp32 arithmetic; results equal the composition's
    to fp32 rounding (different summation order)."""
    if x.ndim != 3:
        raise ValueError(f"x must be [B, H, L]; got shape {tuple(x.shape)}")
    B, H, L = x.shape
    K = grid.shape[0]
    if wout.shape[0] != H:
        raise ValueError(f"the filter has {wout.shape[0]} channels, x has {H}")
    HD = wout.shape[1]
    if not (x.is_cuda and siren_conv_fits(B, H, L, K, HD)):
        from .fftconv_hip import causal_fftconv1d_bhl
        return causal_fftconv1d_bhl(x, siren_filter(grid, w0, b0, hidden_w, hidden_b, wout, bout), shortcut)
    from .fftconv_hip import _grad_wanted, _within_budget
    from .layout import channels_first_contiguous
    f = lambda t: None if t is None else t.float().contiguous()  # noqa: E731
    wh = torch.cat([w.float().reshape(-1) for w in hidden_w])
    bh = None if hidden_b is None else torch.cat([b.float().reshape(-1) for b in hidden_b])
    act = siren_mlp_op(f(grid), f(w0), f(b0), wh, bh, len(hidden_w), HD)
    in_dtype = x.dtype
    cdt = in_dtype if in_dtype in _lib.NSQ_DTYPE else torch.float32
    xc = channels_first_contiguous(x.to(cdt))
    sc = None
    if shortcut is not None:
        if shortcut.shape != (H,):
            raise ValueError(f"shortcut must have shape ({H},); got {tuple(shortcut.shape)}")
        sc = shortcut.to(in_dtype).to(cdt).contiguous()
    wo, bo = f(wout), f(bout)
    keep = _grad_wanted(xc, act, wo, bo, sc) and _within_budget(_siren_conv_ws_bytes(B, H, L, K, HD), x.device) > 0
    y, _ = siren_readout_causal_fftconv1d_op(xc, act, wo, bo, sc, keep)
    return y.to(in_dtype)


def siren_grid(cache_L: Sequence[int], cache_m: Sequence[float], seq_lens: Sequence[int], device=None) -> torch.Tensor:
    """Grid ``[*(2 * s - 1 for s in seq_lens), d]`` of the SIREN positional embedding: per axis the central
    ``2 * s - 1`` points of the cache ``linspace(-m, m, 2 L - 1)`` (``kernels_nd.py:754-778, 835-845``)."""
    axes = []
    for L, m, s in zip(cache_L, cache_m, seq_lens):
        full = torch.linspace(-float(m), float(m), 2 * L - 1, device=device, dtype=torch.float32)
        off = L - s
        axes.append(full[off: off + 2 * s - 1])
    return torch.stack(torch.meshgrid(*axes, indexing="ij"), dim=-1)


class _PositionalEmbedding(torch.nn.Module):
    """The SIREN first layer's parameters (``SIRENPositionalEmbeddingND``: ``linear`` ``[E, d]``)."""

    def __init__(self, data_dim: int, embedding_dim: int, L_cache, omega_0: float, use_bias: bool):
        super().__init__()
        self.data_dim, self.embedding_dim, self.omega_0 = data_dim, embedding_dim, omega_0
        self.L_cache = L_cache
        self.L_cache_per_axis = _per_axis(L_cache, data_dim)
        self.linear = torch.nn.Linear(data_dim, embedding_dim, bias=use_bias)
        _siren_init(self.linear, first=True, w0=omega_0)


def _per_axis(L_cache, data_dim: int) -> tuple[int, ...]:
    if isinstance(L_cache, bool):
        raise TypeError("L_cache must be an int or a sequence of ints, not bool")
    t = (int(L_cache),) * data_dim if isinstance(L_cache, int) else tuple(int(v) for v in L_cache)
    if len(t) != data_dim:
        raise ValueError(f"L_cache has {len(t)} entries for data_dim={data_dim}")
    if any(v < 2 for v in t):
        raise ValueError(f"every L_cache entry must be >= 2; got {t}")
    return t


def _siren_init(layer: torch.nn.Linear, first: bool, w0: float) -> None:
    """SIREN uniform init (Sitzmann et al. 2020) with the frequency folded into the bound:
    first layer U(+-2 pi w0 / d), hidden U(+-sqrt(6 / d)); zero bias (``kernels_nd.py:570-614``)."""
    with torch.no_grad():
        d = layer.in_features
        bound = 2.0 * math.pi * w0 / d if first else math.sqrt(6.0 / d)
        layer.weight.uniform_(-bound, bound)
        if layer.bias is not None:
            layer.bias.zero_()


class KernelFiLMGenerator(torch.nn.Module):
    """The FiLM conditioner of ``SIRENKernelND`` (``modules/film.py:75``): a two-layer MLP ``Linear(cond_dim,
    film_hidden_dim) -> GELU -> Linear(film_hidden_dim, num_film_layers * 2 * kernel_hidden_dim)`` whose output,
    split per layer, gives the ``(gamma, beta)`` pairs the generator applies as ``h <- gamma * h + beta``.

    Same constructor arguments, parameter names (``mlp.0``, ``mlp.2``), initialisation (``"identity"``: output weight
    zero, bias gamma = 1 / beta = 0, so FiLM starts as the identity; ``"small_random"``: output weight N(0,
    ``init_std``)) and weight-decay flags (biases never decayed; ``no_weight_decay=True`` excludes the weights too, a
    float puts them in a group with that decay).  It runs on ``[B, cond_dim]`` vectors, a few small torch ops; the
    per-point work it conditions is in the HIP generator kernels."""

    def __init__(self, cond_dim: int, kernel_hidden_dim: int, num_film_layers: int, film_hidden_dim: int = 64,
                 no_weight_decay: bool | float = False, init_type: str = "identity", init_std: float = 1e-4):
        if num_film_layers < 1:
            raise ValueError(f"num_film_layers must be >= 1, got {num_film_layers}")
        super().__init__()
        self.num_film_layers = num_film_layers
        self.kernel_hidden_dim = kernel_hidden_dim
        width = num_film_layers * 2 * kernel_hidden_dim
        self.mlp = torch.nn.Sequential(torch.nn.Linear(cond_dim, film_hidden_dim), torch.nn.GELU(),
                                       torch.nn.Linear(film_hidden_dim, width))
        last = self.mlp[-1]
        with torch.no_grad():
            if init_type == "identity":
                last.weight.zero_()
            elif init_type == "small_random":
                last.weight.normal_(0.0, init_std)
            else:
                raise ValueError(f"Unknown init_type: {init_type!r}. Expected 'identity' or 'small_random'.")
            pattern = torch.cat([torch.ones(kernel_hidden_dim), torch.zeros(kernel_hidden_dim)])
            last.bias.copy_(pattern.repeat(num_film_layers))
        for m in self.mlp.modules():
            if isinstance(m, torch.nn.Linear) and m.bias is not None:
                m.bias._no_weight_decay = True
        if isinstance(no_weight_decay, float):
            for prm in self.parameters():
                if not getattr(prm, "_no_weight_decay", False):
                    prm._weight_decay = no_weight_decay
        elif no_weight_decay:
            for prm in self.parameters():
                prm._no_weight_decay = True

    def flop_count(self) -> int:
        """Multiply-add count of one sample's MLP, times two, plus the GELU (``film.py`` counts it this way)."""
        a, b = self.mlp[0], self.mlp[2]
        return 2 * a.in_features * a.out_features + a.out_features + 2 * b.in_features * b.out_features

    def forward(self, conditioning: torch.Tensor) -> list[tuple[torch.Tensor, torch.Tensor]]:
        """``conditioning [B, cond_dim]`` -> ``num_film_layers`` pairs ``(gamma [B, HD], beta [B, HD])``, shallowest
        layer first."""
        out = self.mlp(conditioning)
        return [tuple(c.chunk(2, dim=-1)) for c in out.chunk(self.num_film_layers, dim=-1)]


def _build_film(film_cfg) -> torch.nn.Module:
    """The FiLM generator from ``film_cfg``: a module (used as is), a dict of :class:`KernelFiLMGenerator` arguments, or
    a zero-argument factory (such as a lazy config's instantiation)."""
    if isinstance(film_cfg, torch.nn.Module):
        return film_cfg
    if isinstance(film_cfg, dict):
        return KernelFiLMGenerator(**film_cfg)
    if callable(film_cfg):
        return film_cfg()
    raise TypeError(f"film_cfg must be a module, a dict of KernelFiLMGenerator arguments or a factory; got "
                    f"{type(film_cfg).__name__}")


class HipSIRENKernelND(torch.nn.Module):
    """``SIRENKernelND`` (``kernels_nd.py:876``) with the hidden stack in one HIP kernel.

    Same constructor arguments, parameter names and init (state dicts load either way), same
    ``forward(seq_lens) -> (kernel [1, *grid, out_dim], grid [1, *grid, data_dim])``.  ``kernel_bhl``
    gives the channel-first ``[1, out_dim, *grid]`` filter directly (optionally only the causal half in
    1D, the points ``CKConvND`` keeps), which is the layout the HIP FFT convs read.
    """

    def __init__(self, out_dim: int, data_dim: int, mlp_hidden_dim: int, num_layers: int, embedding_dim: int,
                 omega_0: float, L_cache: int | Sequence[int], use_bias: bool, hidden_omega_0: float = 1.0,
                 film_cfg=None, film_after_pos_embed: bool = False):
        super().__init__()
        self.film_after_pos_embed = bool(film_after_pos_embed)
        if film_after_pos_embed:
            assert embedding_dim == mlp_hidden_dim, (
                f"film_after_pos_embed requires embedding_dim == mlp_hidden_dim, got {embedding_dim} != "
                f"{mlp_hidden_dim}")
        if num_layers < 2:
            raise ValueError(f"num_layers must be >= 2; got {num_layers}")
        self.out_dim, self.data_dim, self.mlp_hidden_dim = out_dim, data_dim, mlp_hidden_dim
        self.num_layers, self.embedding_dim = num_layers, embedding_dim
        self.omega_0, self.hidden_omega_0 = float(omega_0), float(hidden_omega_0)
        self.L_cache = L_cache
        self.L_cache_per_axis = _per_axis(L_cache, data_dim)
        self.positional_embedding = _PositionalEmbedding(data_dim, embedding_dim, L_cache, omega_0, use_bias)
        self.hidden_linears = torch.nn.ModuleList(
            [torch.nn.Linear(embedding_dim, mlp_hidden_dim, bias=use_bias)]
            + [torch.nn.Linear(mlp_hidden_dim, mlp_hidden_dim, bias=use_bias) for _ in range(num_layers - 2)])
        self.out_linear = torch.nn.Linear(mlp_hidden_dim, out_dim, bias=use_bias)
        for lin in self.hidden_linears:
            _siren_init(lin, first=False, w0=self.hidden_omega_0)
        _siren_init(self.out_linear, first=False, w0=self.hidden_omega_0)
        with torch.no_grad():  # Wang init of the readout: unit initial energy whatever the grid volume
            self.out_linear.weight.mul_(math.sqrt(1.0 / math.prod(self.L_cache_per_axis)))
        self.num_film_layers = len(self.hidden_linears)
        self.film_generator = None
        if film_cfg is not None:
            self.film_generator = _build_film(film_cfg)
            expected = len(self.hidden_linears) + int(self.film_after_pos_embed)
            if self.film_generator.num_film_layers != expected:
                raise ValueError(
                    f"film_generator.num_film_layers={self.film_generator.num_film_layers} does not match expected "
                    f"{expected} (len(hidden_linears)={len(self.hidden_linears)} + "
                    f"int(film_after_pos_embed)={int(self.film_after_pos_embed)})")
        # grid cache geometry: per-axis extent and limit; the step of the first cache is kept on growth
        self._cache_m = (1.0,) * data_dim
        self.step_sizes = tuple(1.0 / (L - 1) for L in self.L_cache_per_axis)

    def _grid(self, seq_lens: Sequence[int]) -> torch.Tensor:
        """The embedding's grid for ``seq_lens``; an axis longer than the cache grows every axis's cache as
        ``_maybe_extend_grid_cache`` does (``kernels_nd.py:780-815``): ``L <- max(L, s)``,
        ``m <- 1 + step * (L_new - L_old)`` with the original step."""
        assert len(seq_lens) == self.data_dim, f"seq_lens must be of length {self.data_dim}"
        if any(s > L for s, L in zip(seq_lens, self.L_cache_per_axis)):
            new_L = tuple(max(L, s) for L, s in zip(self.L_cache_per_axis, seq_lens))
            self._cache_m = tuple(1.0 + st * (nl - L) for L, nl, st in zip(self.L_cache_per_axis, new_L,
                                                                           self.step_sizes))
            self.L_cache_per_axis = new_L
        return siren_grid(self.L_cache_per_axis, self._cache_m, seq_lens, self.out_linear.weight.device)

    def _filter(self, pts: torch.Tensor, conditioning: torch.Tensor | None = None) -> torch.Tensor:
        """``[nb, H, G]``: one filter (nb = 1), or one per sample of ``conditioning`` when the generator has FiLM."""
        pe = self.positional_embedding.linear
        hb = [lin.bias for lin in self.hidden_linears] if self.hidden_linears[0].bias is not None else None
        hw = [lin.weight for lin in self.hidden_linears]
        if conditioning is not None and self.film_generator is not None:
            film_params = self.film_generator(conditioning)
            return siren_film_filter(pts, pe.weight, pe.bias, hw, hb, self.out_linear.weight, self.out_linear.bias,
                                     film_params, self.film_after_pos_embed)
        return siren_filter(pts, pe.weight, pe.bias, hw, hb, self.out_linear.weight, self.out_linear.bias)[None]

    def forward(self, seq_lens: tuple[int, ...], conditioning: torch.Tensor | None = None):
        """``(kernel [1|B, *grid, out_dim], grid [1, *grid, data_dim])``: the kernel is a view of the channel-first
        filter (``kernel.permute`` back to ``[1|B, out_dim, *grid]`` is contiguous); per sample (``B``) when the
        generator has FiLM and ``conditioning [B, cond_dim]`` is given (``kernels_nd.py:1149-1190``)."""
        grid = self._grid(seq_lens)
        shape = grid.shape[:-1]
        k = self._filter(grid.reshape(-1, self.data_dim), conditioning)  # [nb, H, G]
        kernel = k.reshape(k.shape[0], self.out_dim, *shape).movedim(1, -1)
        return kernel, grid.unsqueeze(0)

    def kernel_bhl(self, seq_lens: tuple[int, ...], causal: bool = False,
                   conditioning: torch.Tensor | None = None) -> torch.Tensor:
        """Channel-first filter ``[1|B, out_dim, *grid]``; ``causal`` (1D): only the points ``kernel_len // 2 ..``
        that ``CKConvND``'s causal crop keeps (``ckconv_nd.py:1159-1164``); per sample with FiLM conditioning."""
        grid = self._grid(seq_lens)
        if causal:
            assert self.data_dim == 1, "the causal crop is 1D"
            grid = grid[grid.shape[0] // 2:]
        shape = grid.shape[:-1]
        k = self._filter(grid.reshape(-1, self.data_dim), conditioning)
        return k.reshape(k.shape[0], self.out_dim, *shape)

    def causal_fftconv1d(self, x: torch.Tensor, shortcut: torch.Tensor | None = None,
                         conditioning: torch.Tensor | None = None) -> torch.Tensor:
        """``CKConvND``'s causal 1D conv with this generator's filter and an identity mask (``ckconv_nd.py:1149-1164``
        then ``fftconv.py:546-600``): ``x [B, out_dim, L]`` convolved with the filter at the ``L`` causal points of
        the ``2L - 1`` grid, plus ``shortcut * x``; equal to ``causal_fftconv1d_bhl(x, self.kernel_bhl((L,), causal=
        True), shortcut)``.  Without FiLM conditioning the filter and its gradient never reach HBM where the shape
        takes the 4-step plan (:func:`siren_causal_fftconv1d`); with it, the per-sample filters are formed and
        convolved."""
        assert self.data_dim == 1, "the causal conv is 1D"
        L = x.shape[-1]
        grid = self._grid((L,))
        pts = grid[grid.shape[0] // 2:].reshape(-1, 1)
        if conditioning is not None and self.film_generator is not None:
            from .fftconv_hip import causal_fftconv1d_bhl
            return causal_fftconv1d_bhl(x, self._filter(pts, conditioning), shortcut)
        pe = self.positional_embedding.linear
        hb = [lin.bias for lin in self.hidden_linears] if self.hidden_linears[0].bias is not None else None
        return siren_causal_fftconv1d(x, pts, pe.weight, pe.bias, [lin.weight for lin in self.hidden_linears], hb,
                                      self.out_linear.weight, self.out_linear.bias, shortcut)
