"""How the integrated EMA is scheduled and where its shadows are kept.

``EMAConfig`` is the public configuration type (its fields, defaults and the
per-step decay of each schedule are the reference's contract,
ema/config.py:13-144). Three schedules exist: a constant decay, a decay moved
linearly to a final value over a number of steps, and the power schedule of
Karras et al. (EDM2), ``(1 - 1/n) ** (gamma + 1)`` at EMA step ``n`` under a
cap, whose average spans a fixed share of the steps taken so far.
"""

from __future__ import annotations

from collections.abc import Callable
from contextlib import AbstractContextManager, nullcontext
from dataclasses import dataclass
from enum import Enum

__all__ = ["EMAConfig", "EMADevice", "EMASchedule", "ProfileRegion", "no_profile"]

# Wraps a piece of EMA work in a named region (a profiler hook, for instance).
ProfileRegion = Callable[[str], AbstractContextManager[object]]


def no_profile(name: str) -> AbstractContextManager[object]:
    """A ``ProfileRegion`` that marks nothing."""
    del name
    return nullcontext()


class EMADevice(Enum):
    """The memory that holds the shadows."""

    GPU = "gpu"
    CPU = "cpu"


class EMASchedule(Enum):
    """The rule that gives each step's decay."""

    CONSTANT = "constant"
    LINEAR_RAMP = "linear_ramp"
    POWER = "power"


def _in_unit_interval(value: float) -> bool:
    return 0.0 <= value < 1.0


@dataclass(frozen=True)
class EMAConfig:
    """Schedule and placement of the integrated EMA.

    Attributes:
        decay: The decay of each step, in [0, 1); the upper bound of the power
            schedule's decay.
        device: GPU or CPU shadows.
        pin_memory: For CPU shadows, allocate them and their staging copies in
            page-locked memory.
        update_every_n_steps: Cadence of the updates (>= 1); each update uses
            the decay to the power n, so the half-life in optimizer steps does
            not change with n.
        start_step: Optimizer step at which the shadows are first set to the
            live weights; nothing happens before it. 0: at the first update.
        decay_final: Target of a linear ramp of the decay, or None.
        decay_ramp_steps: Length of that ramp in optimizer steps (given
            together with ``decay_final``).
        power_gamma: Exponent of the power schedule (> 0), or None; cannot be
            combined with a ramp.

    Raises:
        ValueError: For a value out of range, a ramp given halfway, or a ramp
            together with ``power_gamma``.
    """

    decay: float = 0.9999
    device: EMADevice = EMADevice.GPU
    pin_memory: bool = True
    update_every_n_steps: int = 1
    start_step: int = 0
    decay_final: float | None = None
    decay_ramp_steps: int | None = None
    power_gamma: float | None = None

    def __post_init__(self) -> None:
        problems = [
            (self.update_every_n_steps <= 0, "update_every_n_steps must be 1 or more"),
            (self.start_step < 0, "start_step cannot be negative"),
            (not _in_unit_interval(self.decay), "decay must be in [0, 1)"),
            ((self.decay_final is None) != (self.decay_ramp_steps is None),
             "decay_final and decay_ramp_steps go together: give both or neither"),
            (self.decay_final is not None and not _in_unit_interval(self.decay_final),
             "decay_final must be in [0, 1)"),
            (self.decay_ramp_steps is not None and self.decay_ramp_steps <= 0,
             "decay_ramp_steps must be 1 or more"),
            (self.power_gamma is not None and self.decay_final is not None,
             "a power schedule (power_gamma) and a linear ramp (decay_final) are mutually exclusive"),
            (self.power_gamma is not None and not self.power_gamma > 0.0,
             "power_gamma must be positive (above zero)"),
        ]
        for failed, message in problems:
            if failed:
                raise ValueError(f"EMAConfig.{message}")

    @property
    def schedule(self) -> EMASchedule:
        """The schedule the fields describe."""
        if self.power_gamma is not None:
            return EMASchedule.POWER
        return EMASchedule.CONSTANT if self.decay_final is None else EMASchedule.LINEAR_RAMP

    def decay_at_step(self, step_count: int) -> float:
        """The decay at EMA step ``step_count``.

        Constant: ``decay``. Linear ramp: from ``decay`` to ``decay_final``,
        reached at ``decay_ramp_steps`` and held after. Power: 0 at step 0, then
        ``min(decay, (1 - 1 / step_count) ** (power_gamma + 1))``.

        Raises:
            ValueError: For a negative ``step_count``.
        """
        if step_count < 0:
            raise ValueError("decay_at_step needs a step count of zero or more")
        kind = self.schedule
        if kind is EMASchedule.CONSTANT:
            return self.decay
        if kind is EMASchedule.LINEAR_RAMP:
            assert self.decay_final is not None and self.decay_ramp_steps is not None
            share = min(1.0, step_count / self.decay_ramp_steps)
            return self.decay + share * (self.decay_final - self.decay)
        assert self.power_gamma is not None
        if step_count == 0:
            return 0.0
        return min(self.decay, (1.0 - 1.0 / step_count) ** (self.power_gamma + 1.0))
