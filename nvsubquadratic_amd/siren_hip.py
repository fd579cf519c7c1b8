r"""HIP implicit filter generation: the SIREN MLP of ``SIRENKernelND`` on the matrix cores (row F1).

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

Not covered: FiLM conditioning (``film_cfg``), which raises ``NotImplementedError``; hidden and
embedding widths other than 16, 32, 64 or 128 (raised by the library).
"""

from __future__ import annotations

import math
from collections.abc import Sequence
from typing import Optional

import torch
from torch.library import custom_op

from . import _lib

__all__ = ["HipSIRENKernelND", "siren_filter", "siren_filter_op", "siren_grid"]


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
    lib = _lib.get_lib()
    G, d = grid.shape
    H, HD = wout.shape
    E = w0.shape[0]
    dev = grid.device
    if gk.stride(1) != 1:
        gk = gk.contiguous()
    gact, gwout, gbout = _readout_backward(gk, act, wout, has_bout)
    gw0, gwh = torch.empty_like(w0), torch.empty_like(wh)
    gb0 = torch.empty(E if _has(b0) else 0, device=dev)
    gbh = torch.empty(nh * HD if _has(bh) else 0, device=dev)
    need = lib.nsq_siren_mlp_bwd_workspace_bytes(G, d, E, nh, HD)
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    _lib.check(lib.nsq_siren_mlp_bwd(gact.data_ptr(), gact.stride(0), gact.stride(1), grid.data_ptr(), G, d,
                                     w0.data_ptr(), _opt(b0), E, wh.data_ptr(), _opt(bh), nh, HD, gw0.data_ptr(),
                                     _opt(gb0), gwh.data_ptr(), _opt(gbh), ws.data_ptr(), ws.numel(),
                                     _lib.stream_ptr(dev)))
    return gw0, gb0, gwh, gbh, gwout, gbout


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


def siren_filter(grid: torch.Tensor, w0: torch.Tensor, b0: torch.Tensor | None, hidden_w: Sequence[torch.Tensor],
                 hidden_b: Sequence[torch.Tensor] | None, wout: torch.Tensor, bout: torch.Tensor | None) -> torch.Tensor:
    """Functional form: filter ``[H, G]`` (float32) at the ``G`` points of ``grid [G, d]``.

    ``hidden_w[i]`` is the weight of hidden linear ``i`` (``[HD, E]`` then ``[HD, HD]``), ``hidden_b``
    their biases (None: no biases); every weight is read as float32, as the reference computes.  The
    hidden stack runs in ``nsq_siren_mlp_fwd``, the readout in ``nsq_siren_readout_fwd``; the readout's
    gradients are two GEMMs (``K = H`` and, with the bias as the ones row of ``act``, ``K = G``)."""
    f = lambda t: None if t is None else t.float().contiguous()  # noqa: E731
    wh = torch.cat([w.float().reshape(-1) for w in hidden_w])
    bh = None if hidden_b is None else torch.cat([b.float().reshape(-1) for b in hidden_b])
    return siren_filter_op(f(grid), f(w0), f(b0), wh, bh, f(wout), f(bout), len(hidden_w))[0]


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
        if film_cfg is not None or film_after_pos_embed:
            raise NotImplementedError("fft_backend='hip' SIREN filters: FiLM conditioning is not fused")
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
        self.film_generator = None
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

    def _filter(self, pts: torch.Tensor) -> torch.Tensor:
        pe = self.positional_embedding.linear
        hb = [lin.bias for lin in self.hidden_linears] if self.hidden_linears[0].bias is not None else None
        return siren_filter(pts, pe.weight, pe.bias, [lin.weight for lin in self.hidden_linears], hb,
                            self.out_linear.weight, self.out_linear.bias)

    def forward(self, seq_lens: tuple[int, ...], conditioning: torch.Tensor | None = None):
        """``(kernel [1, *grid, out_dim], grid [1, *grid, data_dim])``: the kernel is a view of the
        channel-first filter (``kernel.permute`` back to ``[1, out_dim, *grid]`` is contiguous)."""
        if conditioning is not None:
            raise NotImplementedError("fft_backend='hip' SIREN filters: FiLM conditioning is not fused")
        grid = self._grid(seq_lens)
        shape = grid.shape[:-1]
        k = self._filter(grid.reshape(-1, self.data_dim))  # [H, G]
        kernel = k.reshape(1, self.out_dim, *shape).movedim(1, -1)
        return kernel, grid.unsqueeze(0)

    def kernel_bhl(self, seq_lens: tuple[int, ...], causal: bool = False) -> torch.Tensor:
        """Channel-first filter ``[1, out_dim, *grid]``; ``causal`` (1D): only the points
        ``kernel_len // 2 ..`` that ``CKConvND``'s causal crop keeps (``ckconv_nd.py:1159-1164``)."""
        grid = self._grid(seq_lens)
        if causal:
            assert self.data_dim == 1, "the causal crop is 1D"
            grid = grid[grid.shape[0] // 2:]
        shape = grid.shape[:-1]
        return self._filter(grid.reshape(-1, self.data_dim)).reshape(1, self.out_dim, *shape)
