"""EMA schedule and placement (reference: src/dionw/ema/config.py:13-144)."""

from __future__ import annotations

from collections.abc import Callable
from contextlib import AbstractContextManager, nullcontext
from dataclasses import dataclass
from enum import Enum

__all__ = ["EMAConfig", "EMADevice", "EMASchedule", "ProfileRegion", "no_profile"]

# A named profiling region around EMA work.
ProfileRegion = Callable[[str], AbstractContextManager[object]]


def no_profile(name: str) -> AbstractContextManager[object]:
    """The default ``ProfileRegion``: nothing."""
    del name
    return nullcontext()


class EMADevice(Enum):
    """Where EMA shadows live."""

    GPU = "gpu"
    CPU = "cpu"


class EMASchedule(Enum):
    """How the per-step decay evolves."""

    CONSTANT = "constant"
    LINEAR_RAMP = "linear_ramp"
    POWER = "power"


@dataclass(frozen=True)
class EMAConfig:
    """EMA schedule and placement.

    Attributes:
        decay: Per-step decay in [0, 1) (the power schedule's cap).
        device: Where shadows live.
        pin_memory: Pin CPU shadows and staging buffers (CPU EMA).
        update_every_n_steps: Update cadence (>= 1); the decay is raised to n.
        start_step: First optimizer step that copies the live weights into the
            shadows (0: the first update).
        decay_final: End of a linear ramp, or None.
        decay_ramp_steps: Steps of the ramp; set with ``decay_final``.
        power_gamma: Exponent of the power schedule (> 0), or None.

    Raises:
        ValueError: For out-of-range values, a half-specified ramp, or a ramp
            combined with ``power_gamma``.
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
        if self.update_every_n_steps <= 0:
            raise ValueError("EMAConfig.update_every_n_steps must be positive")
        if self.start_step < 0:
            raise ValueError("EMAConfig.start_step must be non-negative")
        if not 0.0 <= self.decay < 1.0:
            raise ValueError("EMAConfig.decay must be in [0, 1)")
        if (self.decay_final is None) != (self.decay_ramp_steps is None):
            raise ValueError("EMAConfig.decay_final and decay_ramp_steps must be set together")
        if self.decay_final is not None and not 0.0 <= self.decay_final < 1.0:
            raise ValueError("EMAConfig.decay_final must be in [0, 1)")
        if self.decay_ramp_steps is not None and self.decay_ramp_steps <= 0:
            raise ValueError("EMAConfig.decay_ramp_steps must be positive")
        if self.power_gamma is not None:
            if self.decay_final is not None:
                raise ValueError("EMAConfig.power_gamma and the decay_final ramp are exclusive")
            if not self.power_gamma > 0.0:
                raise ValueError("EMAConfig.power_gamma must be positive")

    @property
    def schedule(self) -> EMASchedule:
        """The schedule the set fields select."""
        if self.power_gamma is not None:
            return EMASchedule.POWER
        if self.decay_final is not None:
            return EMASchedule.LINEAR_RAMP
        return EMASchedule.CONSTANT

    def decay_at_step(self, step_count: int) -> float:
        """The per-step decay at EMA step ``step_count``.

        CONSTANT: ``decay``. LINEAR_RAMP: ``decay`` moved linearly to
        ``decay_final`` over ``decay_ramp_steps``. POWER: ``(1 - 1/n) **
        (gamma + 1)`` capped at ``decay`` (0 at n = 0).

        Raises:
            ValueError: If ``step_count`` is negative.
        """
        if step_count < 0:
            raise ValueError("step_count must be non-negative")
        schedule = self.schedule
        if schedule is EMASchedule.CONSTANT:
            return self.decay
        if schedule is EMASchedule.LINEAR_RAMP:
            assert self.decay_final is not None and self.decay_ramp_steps is not None
            progress = min(1.0, step_count / self.decay_ramp_steps)
            return self.decay + (self.decay_final - self.decay) * progress
        assert self.power_gamma is not None
        if step_count == 0:
            return 0.0
        return min(self.decay, (1.0 - 1.0 / step_count) ** (self.power_gamma + 1.0))
