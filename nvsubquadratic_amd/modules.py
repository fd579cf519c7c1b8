"""The Hyena short-conv slot as an ``nn.Conv1d`` on the HIP backend.

Hyena accepts any ``nn.Conv1d`` for its short convolution
(``nvsubquadratic/modules/hyena_nd.py:258-271`` checks the type), and the
reference fills the slot with ``SubqOpsCausalConv1d``
(``nvsubquadratic/modules/subq_ops_causal_conv1d.py:36-83``).
:class:`HipCausalConv1d` takes the same constructor arguments and keeps the
same parameters (``weight`` of shape ``[C, 1, K]``, optional ``bias`` of shape
``[C]``), so checkpoints move between the two unchanged; its forward runs
:func:`nvsubquadratic_amd.causal_conv1d_hip.causal_conv1d`.
"""

from __future__ import annotations

import torch

from .causal_conv1d_hip import causal_conv1d


__all__ = ["HipCausalConv1d"]

_ACTIVATIONS = ("identity", "silu")


class HipCausalConv1d(torch.nn.Conv1d):
    """Per-channel causal convolution: output n sees inputs n-K+1 .. n of its own channel."""

    def __init__(
        self,
        in_channels: int,
        out_channels: int,
        kernel_size: int,
        *,
        groups: int,
        bias: bool = False,
        activation: str = "identity",
    ) -> None:
        """
        Args:
            in_channels: C, the number of channels.
            out_channels: also C; each channel has its own filter.
            kernel_size: K, the filter length (1 <= K <= 256 for the HIP kernels).
            groups: also C (one group per channel).
            bias: add a learned per-channel offset before the activation.
            activation: ``"identity"`` or ``"silu"``, fused into the kernel's output.

        Raises:
            ValueError: when the three channel arguments differ (the layer is
                depthwise-only) or the activation is not one of the two above.
        """
        if groups != in_channels or out_channels != in_channels:
            raise ValueError(
                f"HipCausalConv1d is depthwise-only (one filter per channel), so in_channels, out_channels and "
                f"groups have to agree; received in_channels={in_channels}, out_channels={out_channels}, "
                f"groups={groups}."
            )
        if activation not in _ACTIVATIONS:
            raise ValueError(f"unsupported activation {activation!r}; choose one of {_ACTIVATIONS}.")
        super().__init__(in_channels, out_channels, kernel_size, groups=groups, bias=bias, padding=0)
        self.activation = activation

    def forward(self, input: torch.Tensor) -> torch.Tensor:  # type: ignore[override]
        """``input`` is ``[B, C, L]``; returns ``[B, C, L]`` in the input's dtype."""
        # The parameter keeps nn.Conv1d's [C, 1, K] layout; the op takes one filter row per channel.
        return causal_conv1d(input, self.weight[:, 0, :], self.bias, self.activation)
