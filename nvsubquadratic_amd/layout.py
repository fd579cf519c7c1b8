r"""Channels-last to channels-first layout change on the HIP backend.

The reference's ``_w_reshape`` / ``_blh`` wrappers (``nvsubquadratic/ops/fftconv.py:163-232, 449-538``,
``nvsubquadratic/ops/fftconv_custom.py:338-359``) call the channels-first op on ``rearrange(x, "b l h -> b h
l")``, a view that the op then materialises (``.contiguous()``), and hand the result back as a view; their
backward does the same with the incoming gradient.  torch's permute-copy of such a view runs at about 1 TB/s
for 16-bit elements on MI355X, a fifth of a plain copy.  :func:`channels_first_contiguous` moves a
channels-last view through ``nsq_batched_transpose`` (64 x 64 LDS tiles, 16-byte accesses) instead, as a
``torch.library`` custom op whose backward is the inverse transpose.
"""

from __future__ import annotations

import torch
from torch.library import custom_op

from . import _lib

__all__ = ["channels_first_contiguous", "transpose_fits", "transpose_inner_op"]


@custom_op("nsq_hip::transpose_inner", mutates_args=())
def transpose_inner_op(x: torch.Tensor) -> torch.Tensor:
    """``[B, R, C]`` (contiguous) -> ``[B, C, R]`` contiguous, element size 2 or 4 bytes."""
    lib = _lib.get_lib()
    _lib.check_device(x)
    B, R, C = x.shape
    out = torch.empty(B, C, R, dtype=x.dtype, device=x.device)
    if x.numel():
        _lib.check(lib.nsq_batched_transpose(x.data_ptr(), out.data_ptr(), x.element_size(), B, R, C,
                                             _lib.stream_ptr(x.device)))
    return out


@transpose_inner_op.register_fake
def _(x):
    B, R, C = x.shape
    return x.new_empty(B, C, R)


def _transpose_backward(ctx, g):
    return transpose_inner_op(g.contiguous())


transpose_inner_op.register_autograd(_transpose_backward, setup_context=lambda ctx, inputs, output: None)


def transpose_fits(B: int, C: int) -> bool:
    """Whether ``nsq_batched_transpose`` takes a ``[B, R, C]`` batch: the batch on grid.z and the column tiles
    (64 channels each) on grid.y, at most 65535 each; the row tiles sit on grid.x (2^31 - 1), so R is free."""
    return B <= 65535 and -(-C // 64) <= 65535


def channels_first_contiguous(t: torch.Tensor) -> torch.Tensor:
    """``t`` ``[B, H, *S]`` as a contiguous tensor.  A channels-last view (``t.movedim(1, -1)`` contiguous, as a
    ``_w_reshape`` / ``_blh`` wrapper's ``rearrange`` or the gradient of its output leaves it) moves through
    ``nsq_batched_transpose``; any other layout goes through ``Tensor.contiguous``."""
    if t.is_contiguous() or t.dim() < 3 or not t.is_cuda or t.element_size() not in (2, 4):
        return t.contiguous()
    m = t.movedim(1, -1)
    B, H = t.shape[0], t.shape[1]
    if not m.is_contiguous() or not transpose_fits(B, H) or t.numel() == 0:
        return t.contiguous()
    return transpose_inner_op(m.reshape(B, -1, H)).view(t.shape)
