"""Evaluation with the EMA weights: the live weights set aside and put back.

``WeightSwap`` holds the live values of the parameters whose shadows replaced
them. Which parameters swap is decided by ``swap_plan``: every trainable
parameter of the optimizer, or those of a given module, which must then share
parameters with the optimizer and hold no trainable parameter outside it; the
swap is all-or-nothing (every chosen parameter has a shadow, or none has:
before the first update nothing is swapped). Behaviour and messages follow the
reference (ema/_swap.py:22-101, ema/mixin.py:251-308).
"""

from __future__ import annotations

from collections.abc import Mapping, Sequence

import torch
from torch import Tensor, nn

from dionw_amd.ema._keys import EMA_SHADOW

__all__ = ["WeightSwap", "swap_plan"]


def swap_plan(model: nn.Module | None, managed: Sequence[nn.Parameter],
              state: Mapping[Tensor, Mapping[str, object]], context: str
              ) -> list[tuple[nn.Parameter, Tensor]]:
    """The (parameter, shadow) pairs a swap applies; empty before any shadow.

    Raises:
        ValueError: If there is nothing to swap, or ``model`` shares no
            parameter with the optimizer or has trainable ones outside it.
        TypeError: If a shadow is not a tensor.
        RuntimeError: If only some of the chosen parameters have shadows.
    """
    if not managed:
        raise ValueError("No parameters to swap: the optimizer holds no trainable ones")
    chosen: Sequence[nn.Parameter] = managed
    if model is not None:
        ids = {id(p) for p in managed}
        inside = [p for p in model.parameters() if id(p) in ids]
        strangers = [p for p in model.parameters() if id(p) not in ids and p.requires_grad]
        if strangers:
            raise ValueError(f"{context}: {len(strangers)} trainable parameters of the model "
                             "given to the EMA swap lie outside the optimizer")
        if not inside:
            raise ValueError(f"{context}: the model given to the EMA swap has no "
                             "optimizer-managed parameters")
        chosen = inside
    pairs = []
    for param in chosen:
        shadow = state.get(param, {}).get(EMA_SHADOW)
        if shadow is None:
            continue
        if not isinstance(shadow, Tensor):
            raise TypeError(f"{context}: a stored EMA shadow is not a tensor")
        pairs.append((param, shadow))
    if pairs and len(pairs) != len(chosen):
        raise RuntimeError(f"{context}: only {len(pairs)} of {len(chosen)} parameters have an "
                           "initialized shadow; a partial swap would mix live and EMA weights")
    return pairs


class WeightSwap:
    """Live weights set aside while the EMA weights are in the parameters."""

    def __init__(self) -> None:
        self._held: dict[int, tuple[nn.Parameter, Tensor]] = {}

    @property
    def active(self) -> bool:
        """Whether EMA weights are in the parameters."""
        return bool(self._held)

    @torch.no_grad()
    def apply(self, pairs: Sequence[tuple[nn.Parameter, Tensor]]) -> bool:
        """Set the live weights aside and copy the shadows in.

        Raises:
            RuntimeError: If a swap is already active.
        """
        if self._held:
            raise RuntimeError("the EMA weights are already swapped in; restore the live weights first")
        for param, shadow in pairs:
            self._held[id(param)] = (param, param.data.clone())
            param.data.copy_(shadow.to(device=param.device, dtype=param.dtype))
        return bool(pairs)

    @torch.no_grad()
    def undo(self) -> None:
        """Copy the live weights back."""
        for param, live in self._held.values():
            param.data.copy_(live)
        self._held.clear()
