"""``IntegratedEMAOptimizer``: the EMA as an optimizer mixin.

List it before a concrete optimizer (``class X(IntegratedEMAOptimizer,
torch.optim.AdamW)``) and call ``_init_integrated_ema`` at the end of
``__init__``; the concrete optimizer must create a parameter's state no later
than its first step, since shadows are made for parameters with state.

Around every step the mixin runs the EMA cadence (``_ema_cadence``: refuse to
step while EMA weights are swapped in, advance the schedule, then after the
concrete update move each due shadow). A subclass with its own ``step`` uses
the same context manager. Checkpoints carry the shadows in the per-parameter
state and the schedule position as the top-level ``_ema_step_count``; the
CPU EMA's staging buffers and flags stay out (reference ema/mixin.py:87-308).
"""

from __future__ import annotations

from collections.abc import Callable, Iterator, Mapping
from contextlib import contextmanager
from typing import Any

import torch
from torch import Tensor
from torch.optim import Optimizer

from dionw_amd.ema._keys import (
    EMA_INITIALIZED,
    EMA_KEY_PREFIX,
    EMA_SCRATCH_KEYS,
    EMA_SHADOW,
    EMA_STEP_COUNT_KEY,
)
from dionw_amd.ema._swap import WeightSwap, swap_plan
from dionw_amd.ema.config import EMAConfig, ProfileRegion
from dionw_amd.ema.tracker import OptimizerIntegratedEMA

__all__ = ["IntegratedEMAOptimizer"]


def _carries_ema(state_dict: Mapping[str, Any]) -> bool:
    return EMA_STEP_COUNT_KEY in state_dict or any(
        key.startswith(EMA_KEY_PREFIX) for entry in state_dict["state"].values() for key in entry)


def _split_ema(state_dict: Mapping[str, Any]) -> tuple[dict[str, Any], Any]:
    """The state dict without EMA entries, and the saved step count."""
    core = {k: v for k, v in state_dict.items() if k != EMA_STEP_COUNT_KEY}
    core["state"] = {index: {k: v for k, v in entry.items() if not k.startswith(EMA_KEY_PREFIX)}
                     for index, entry in state_dict["state"].items()}
    return core, state_dict.get(EMA_STEP_COUNT_KEY)


class IntegratedEMAOptimizer(Optimizer):
    """Optimizer mixin that moves an ``OptimizerIntegratedEMA`` after each step."""

    _ema_helper: OptimizerIntegratedEMA | None
    _weight_swap: WeightSwap

    def _init_integrated_ema(self, ema: EMAConfig | None, profile_region: ProfileRegion) -> None:
        """Attach the EMA (None disables it).

        Raises:
            ValueError: If the optimizer has no trainable parameter.
        """
        if not self._trainable():
            raise ValueError(f"{type(self).__name__} has no parameter that requires a gradient")
        self._ema_helper = None if ema is None else OptimizerIntegratedEMA(self, ema,
                                                                            profile_region)
        self._weight_swap = WeightSwap()

    def _trainable(self) -> list[torch.nn.Parameter]:
        return [p for group in self.param_groups for p in group["params"] if p.requires_grad]

    @property
    def ema(self) -> OptimizerIntegratedEMA | None:
        """The attached EMA tracker; None for an optimizer built without EMA."""
        return self._ema_helper

    @contextmanager
    def _ema_cadence(self) -> Iterator[None]:
        """The EMA around one optimizer update: the body is the update.

        Parameters without a gradient keep their value, but their shadows still
        move on the global cadence.

        Raises:
            RuntimeError: If the EMA weights are in the parameters.
        """
        if self._weight_swap.active:
            raise RuntimeError("cannot step while the EMA weights are swapped in; call "
                               "restore_non_ema_weights() before stepping")
        helper = self._ema_helper
        if helper is not None:
            helper.begin_step()
        yield
        if helper is not None and helper.should_update_this_step():
            for param in self._trainable():
                helper.update_param(param)
            helper.finalize_updates()

    @torch.no_grad()
    def step(self, closure: Callable[[], float] | None = None) -> float | None:  # type: ignore[override]
        """The concrete optimizer's step inside the EMA cadence."""
        with self._ema_cadence():
            loss = super().step(closure)
        return loss

    def state_dict(self) -> dict[str, Any]:
        """The optimizer state with the shadows and the EMA step count."""
        helper = self._ema_helper
        if helper is None:
            return super().state_dict()
        helper.flush_pending_updates()
        state = super().state_dict()
        state["state"] = {index: {k: v for k, v in entry.items() if k not in EMA_SCRATCH_KEYS}
                          for index, entry in state["state"].items()}
        state[EMA_STEP_COUNT_KEY] = helper.step_count
        return state

    def load_state_dict(self, state_dict: dict[str, Any]) -> None:
        """Restore the state, then the shadows on the EMA device and the step count.

        Raises:
            ValueError: For EMA state without an EMA, or an EMA without a valid
                saved step count.
        """
        helper = self._ema_helper
        name = type(self).__name__
        if helper is None:
            if _carries_ema(state_dict):
                raise ValueError(
                    f"this {name} checkpoint holds EMA shadows, but the optimizer was built "
                    "without EMA (ema=None): pass the EMAConfig it was saved with, or load a "
                    "state saved without an EMA")
            super().load_state_dict(state_dict)
            return
        helper.flush_pending_updates()
        core, count = _split_ema(state_dict)
        if type(count) is not int or count < 0:
            raise ValueError(f"this {name} checkpoint was saved without an EMA: its "
                             f"{EMA_STEP_COUNT_KEY} is {count!r}, not a count of zero or more")
        super().load_state_dict(core)
        for saved_group, group in zip(state_dict["param_groups"], self.param_groups, strict=True):
            for index, param in zip(saved_group["params"], group["params"], strict=True):
                saved = state_dict["state"].get(index, {})
                if EMA_SHADOW in saved:
                    helper.restore_shadow(param, saved[EMA_SHADOW], saved[EMA_INITIALIZED])
        helper.step_count = count

    @property
    def ema_weights_swapped(self) -> bool:
        """True between ``swap_ema_weights`` and ``restore_non_ema_weights``."""
        return self._weight_swap.active

    @torch.no_grad()
    def swap_ema_weights(self, model: torch.nn.Module | None = None) -> bool:
        """Put the shadows into the parameters, for evaluation; undo with
        ``restore_non_ema_weights`` (``step`` refuses to run until then).

        Args:
            model: Swap only this module's parameters; None swaps all of the
                optimizer's.

        Returns:
            Whether EMA weights went in (False without EMA or before the first
            update).

        Raises:
            RuntimeError: If the EMA weights are in the parameters already.
            ValueError: Without parameters to swap, or for a ``model`` that
                shares none with the optimizer or has trainable ones outside it.
        """
        helper = self._ema_helper
        if helper is None:
            return False
        if self._weight_swap.active:
            raise RuntimeError("the EMA weights are already swapped in; restore the live weights first")
        helper.flush_pending_updates()
        pairs = swap_plan(model, self._trainable(), self.state, type(self).__name__)
        return self._weight_swap.apply(pairs)

    @torch.no_grad()
    def restore_non_ema_weights(self) -> bool:
        """Put the live weights back (False without EMA, else True)."""
        if self._ema_helper is None:
            return False
        self._weight_swap.undo()
        return True

