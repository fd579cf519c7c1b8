"""Module-level drop-ins for the Hyena short-conv slot.

:class:`HipCausalConv1d` mirrors ``SubqOpsCausalConv1d``
(``nvsubquadratic/modules/subq_ops_causal_conv1d.py:36-83``): an
``nn.Conv1d`` subclass (so ``Hyena``'s ``isinstance(short_conv, nn.Conv1d)``
check at ``nvsubquadratic/modules/hyena_nd.py:258-271`` passes) with the same
``weight [C, 1, K]`` / ``bias [C]`` state-dict layout, the same constructor
checks and error messages, running :func:`nvsubquadratic_amd.causal_conv1d_hip.causal_conv1d`.
"""

from __future__ import annotations

import torch

from .causal_conv1d_hip import causal_conv1d


__all__ = ["HipCausalConv1d"]


class HipCausalConv1d(torch.nn.Conv1d):
    """Depthwise causal 1D conv on the gfx950 HIP backend."""

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
        """Build a depthwise causal conv with optional SiLU activation.

        Args:
            in_channels: Channel count (must equal ``out_channels`` and ``groups``).
            out_channels: Output channels (depthwise: same as ``in_channels``).
            kernel_size: Causal kernel length (1..256).
            groups: Must equal ``in_channels`` for depthwise layout.
            bias: Whether to include a per-channel bias.
            activation: ``"identity"`` or ``"silu"`` applied inside the kernel.
        """
        if not (groups == in_channels == out_channels):
            raise ValueError(
                "HipCausalConv1d is depthwise-only: groups must equal "
                f"in_channels must equal out_channels.  Got groups={groups}, "
                f"in_channels={in_channels}, out_channels={out_channels}."
            )
        if activation not in ("identity", "silu"):
            raise ValueError(f"activation must be 'identity' or 'silu'. Got {activation!r}.")
        super().__init__(
            in_channels=in_channels,
            out_channels=out_channels,
            kernel_size=kernel_size,
            groups=groups,
            bias=bias,
            padding=0,
        )
        self.activation = activation

    def forward(self, input: torch.Tensor) -> torch.Tensor:  # type: ignore[override]
        """Run causal depthwise conv; input shape ``[B, C, L]``."""
        # nn.Conv1d depthwise weight is [C, 1, K]; the kernel takes [C, K].
        return causal_conv1d(input, self.weight.squeeze(1), self.bias, self.activation)
