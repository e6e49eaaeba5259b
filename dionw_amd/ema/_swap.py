"""Temporary swaps of the live weights with their EMA shadows.

Reference: src/dionw/ema/_swap.py:22-101.
"""

from __future__ import annotations

from collections.abc import Mapping, MutableMapping, Sequence
from dataclasses import dataclass

import torch
from torch import Tensor

from dionw_amd.ema._keys import EMA_SHADOW

__all__ = ["EmaSwapEntry", "collect_state_ema_swap_entries", "optimizer_managed_ema_swap_params"]


@dataclass(frozen=True)
class EmaSwapEntry:
    """A parameter and its shadow."""

    parameter: torch.nn.Parameter
    shadow: Tensor


def collect_state_ema_swap_entries(
    *, params: Sequence[torch.nn.Parameter], optimizer_state: Mapping[Tensor, object], context: str
) -> tuple[EmaSwapEntry, ...]:
    """Every parameter's shadow, or nothing before the EMA has started.

    Raises:
        ValueError: If ``params`` is empty.
        TypeError: If a shadow is not a tensor.
        RuntimeError: If only some parameters have shadows.
    """
    if not params:
        raise ValueError("No parameters available to swap with EMA weights")
    found: list[EmaSwapEntry] = []
    missing = 0
    for parameter in params:
        entry = optimizer_state.get(parameter)
        shadow = entry.get(EMA_SHADOW) if isinstance(entry, MutableMapping) else None
        if shadow is None:
            missing += 1
        elif not isinstance(shadow, Tensor):
            raise TypeError(f"{context} EMA shadow must be a torch.Tensor")
        else:
            found.append(EmaSwapEntry(parameter, shadow))
    if found and missing:
        raise RuntimeError(
            f"{context} EMA swap found {len(found)} initialized shadows for {len(params)} "
            "parameters. Refusing to mix live and EMA weights."
        )
    return tuple(found)


def optimizer_managed_ema_swap_params(
    *,
    model: torch.nn.Module | None,
    optimizer_params: Sequence[torch.nn.Parameter],
    context: str,
) -> tuple[torch.nn.Parameter, ...]:
    """The parameters to swap: the optimizer's, scoped to ``model`` if given.

    Raises:
        ValueError: Without optimizer parameters, or if ``model`` shares none
            with the optimizer or has trainable parameters outside it.
    """
    if not optimizer_params:
        raise ValueError("No parameters available to swap with EMA weights")
    if model is None:
        return tuple(optimizer_params)
    managed = {id(p) for p in optimizer_params}
    scoped = [p for p in model.parameters() if id(p) in managed]
    outside = sum(1 for p in model.parameters() if id(p) not in managed and p.requires_grad)
    if outside:
        raise ValueError(
            f"{context} EMA swap received a model with {outside} trainable parameters "
            "outside the optimizer."
        )
    if not scoped:
        raise ValueError(f"{context} EMA swap received a model with no optimizer-managed parameters.")
    return tuple(scoped)
