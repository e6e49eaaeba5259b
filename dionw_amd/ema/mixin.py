"""``IntegratedEMAOptimizer``: an optimizer mixin with an integrated EMA.

Reference: src/dionw/ema/mixin.py:38-308. The mixin steps, saves and loads an
``OptimizerIntegratedEMA`` and swaps the live weights with the shadows for
evaluation.
"""

from __future__ import annotations

from collections.abc import Callable, Mapping
from typing import Any

import torch
from torch import Tensor
from torch.optim import Optimizer

from dionw_amd.ema._keys import (
    EMA_INITIALIZED,
    EMA_KEY_PREFIX,
    EMA_PENDING,
    EMA_SCRATCH_KEYS,
    EMA_SHADOW,
    EMA_STEP_COUNT_KEY,
    EMA_TMP_CPU,
)
from dionw_amd.ema._swap import collect_state_ema_swap_entries, optimizer_managed_ema_swap_params
from dionw_amd.ema._update import FP32
from dionw_amd.ema.config import EMAConfig, ProfileRegion
from dionw_amd.ema.tracker import OptimizerIntegratedEMA, new_cpu_staging

__all__ = ["IntegratedEMAOptimizer"]


class IntegratedEMAOptimizer(Optimizer):
    """Optimizer mixin that updates an ``OptimizerIntegratedEMA`` after each step.

    List it before the concrete optimizer and call ``_init_integrated_ema`` at
    the end of ``__init__``; the concrete optimizer must create a parameter's
    state no later than its first step.
    """

    _ema_helper: OptimizerIntegratedEMA | None
    _stored_params: dict[int, Tensor]

    def _init_integrated_ema(self, ema: EMAConfig | None, profile_region: ProfileRegion) -> None:
        """Attach the EMA (None disables it).

        Raises:
            ValueError: If the optimizer has no trainable parameter.
        """
        if not self._iter_trainable_params():
            raise ValueError(f"{type(self).__name__} requires at least one trainable parameter")
        self._ema_helper = None if ema is None else OptimizerIntegratedEMA(self, ema, profile_region)
        self._stored_params = {}

    def _iter_trainable_params(self) -> list[torch.nn.Parameter]:
        return [p for g in self.param_groups for p in g["params"] if p.requires_grad]

    @property
    def ema(self) -> OptimizerIntegratedEMA | None:
        """The EMA, or None when disabled."""
        return self._ema_helper

    @torch.no_grad()
    def step(self, closure: Callable[[], float] | None = None) -> float | None:  # type: ignore[override]
        """The concrete optimizer's step, then the due EMA update.

        Raises:
            RuntimeError: While EMA weights are swapped in.
        """
        if self._stored_params:
            raise RuntimeError(
                "step() while EMA weights are swapped in: call restore_non_ema_weights() first"
            )
        helper = self._ema_helper
        due = False
        if helper is not None:
            helper.begin_step()
            due = helper.should_update_this_step()
        loss = super().step(closure)
        if helper is not None and due:
            for param in self._iter_trainable_params():
                helper.update_param(param)
            helper.finalize_updates()
        return loss

    def state_dict(self) -> dict[str, Any]:
        """The optimizer state with the shadows and the EMA step count."""
        if self._ema_helper is None:
            return super().state_dict()
        self._ema_helper.flush_pending_updates()
        state = super().state_dict()
        state["state"] = {
            index: {k: v for k, v in entry.items() if k not in EMA_SCRATCH_KEYS}
            for index, entry in state["state"].items()
        }
        state[EMA_STEP_COUNT_KEY] = self._ema_helper.step_count
        return state

    def load_state_dict(self, state_dict: dict[str, Any]) -> None:
        """Restore the state, the shadows (on the EMA device) and the step count.

        Raises:
            ValueError: For EMA state without an EMA, or a missing/invalid
                step count with one.
        """
        helper = self._ema_helper
        name = type(self).__name__
        if helper is None:
            carries = EMA_STEP_COUNT_KEY in state_dict or any(
                key.startswith(EMA_KEY_PREFIX)
                for entry in state_dict["state"].values()
                for key in entry
            )
            if carries:
                raise ValueError(
                    f"Checkpoint {name} state carries EMA shadows but the optimizer was built "
                    "without EMA (ema=None). Build it with the saved EMAConfig to continue the "
                    "EMA, or load a fresh optimizer state without the EMA."
                )
            super().load_state_dict(state_dict)
            return
        helper.flush_pending_updates()
        count = state_dict.get(EMA_STEP_COUNT_KEY)
        if type(count) is not int or count < 0:
            raise ValueError(
                f"{name} state has no valid EMA step count ({EMA_STEP_COUNT_KEY}={count!r}): "
                "it was not saved with an EMA"
            )
        stripped = {k: v for k, v in state_dict.items() if k != EMA_STEP_COUNT_KEY}
        stripped["state"] = {
            index: {k: v for k, v in entry.items() if not k.startswith(EMA_KEY_PREFIX)}
            for index, entry in state_dict["state"].items()
        }
        super().load_state_dict(stripped)
        self._restore_shadows(state_dict, helper)
        helper.step_count = count

    def _restore_shadows(self, saved: Mapping[str, Any], helper: OptimizerIntegratedEMA) -> None:
        on_gpu = helper.uses_gpu_shadow
        pin = helper.config.pin_memory and not on_gpu
        for saved_group, group in zip(saved["param_groups"], self.param_groups, strict=True):
            for index, param in zip(saved_group["params"], group["params"], strict=True):
                source = saved["state"].get(index, {})
                if EMA_SHADOW not in source:
                    continue
                shadow = source[EMA_SHADOW]
                if not isinstance(shadow, Tensor):
                    raise TypeError(f"{type(self).__name__} EMA shadow must be a tensor")
                device = param.device if on_gpu else torch.device("cpu")
                state = self.state[param]
                state[EMA_SHADOW] = torch.empty_like(
                    shadow, device=device, dtype=FP32, pin_memory=pin
                ).copy_(shadow)
                state[EMA_INITIALIZED] = source[EMA_INITIALIZED]
                state[EMA_PENDING] = False
                if not on_gpu:
                    state[EMA_TMP_CPU] = new_cpu_staging(param, pin=pin)

    @property
    def ema_weights_swapped(self) -> bool:
        """Whether ``swap_ema_weights`` holds EMA weights in the parameters."""
        return bool(self._stored_params)

    @torch.no_grad()
    def swap_ema_weights(self, model: torch.nn.Module | None = None) -> bool:
        """Swap the parameters with their shadows (undo: ``restore_non_ema_weights``).

        Returns:
            Whether EMA weights were applied (False without EMA or before the
            first update).

        Raises:
            RuntimeError: If EMA weights are already swapped in.
            ValueError: Without parameters to swap, or for a ``model`` that
                shares none with the optimizer or has others.
        """
        if self._ema_helper is None:
            return False
        if self._stored_params:
            raise RuntimeError("EMA weights are already swapped in")
        self._ema_helper.flush_pending_updates()
        context = type(self).__name__
        params = optimizer_managed_ema_swap_params(
            model=model, optimizer_params=self._iter_trainable_params(), context=context
        )
        entries = collect_state_ema_swap_entries(
            params=params, optimizer_state=self.state, context=context
        )
        for entry in entries:
            param = entry.parameter
            self._stored_params[id(param)] = param.data.clone()
            param.data.copy_(entry.shadow.to(device=param.device, dtype=param.dtype))
        return bool(entries)

    @torch.no_grad()
    def restore_non_ema_weights(self) -> bool:
        """Restore the weights saved by ``swap_ema_weights`` (False without EMA)."""
        if self._ema_helper is None:
            return False
        for param in self._iter_trainable_params():
            stored = self._stored_params.get(id(param))
            if stored is not None:
                param.data.copy_(stored)
        self._stored_params.clear()
        return True
