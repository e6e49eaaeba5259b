"""Background worker of CPU EMA: one queued update at a time.

Reference: src/dionw/ema/_cpu_job.py:20-137. A daemon thread waits for the
staged device-to-host copies, then applies every shadow update on the CPU; an
exception in the worker is kept and re-raised by the next wait.
"""

from __future__ import annotations

from dataclasses import dataclass
from threading import Event, Thread
from typing import Any

import torch
from torch import Tensor

from dionw_amd.ema._keys import EMA_EVENT, EMA_INITIALIZED, EMA_PENDING
from dionw_amd.ema._update import FP32, ema_update_

__all__ = ["AsyncCpuEmaItem", "AsyncCpuEmaJob"]


@dataclass
class AsyncCpuEmaItem:
    """One staged CPU update: the state entry, the copy's event (or None),
    the float32 CPU shadow and the staged snapshot.

    Raises:
        ValueError: If the shadow or the snapshot is not on the CPU.
    """

    state: dict[str, Any]
    event: torch.cuda.Event | None
    shadow: Tensor
    tmp_cpu: Tensor

    def __post_init__(self) -> None:
        if self.shadow.device.type != "cpu" or self.tmp_cpu.device.type != "cpu":
            raise ValueError("CPU EMA shadows and staging buffers must be on the CPU")


class AsyncCpuEmaJob:
    """One queued CPU update with copy-ready and update-done barriers."""

    def __init__(
        self, *, items: list[AsyncCpuEmaItem], decay: float, fp32_staging: Tensor | None
    ) -> None:
        """Create the job (not started).

        Raises:
            ValueError: Without items, or if a non-float32 snapshot does not fit
                the staging buffer.
        """
        if not items:
            raise ValueError("AsyncCpuEmaJob requires at least one item")
        largest = max((i.tmp_cpu.numel() for i in items if i.tmp_cpu.dtype != FP32), default=0)
        if largest > (0 if fp32_staging is None else fp32_staging.numel()):
            raise ValueError("CPU EMA FP32 staging buffer is smaller than a snapshot")
        self.items = items
        self.decay = decay
        self.fp32_staging = fp32_staging
        self.copy_ready = Event()
        self.update_done = Event()
        self.exception: BaseException | None = None
        self._thread = Thread(target=self._work, name="dionw_cpu_ema", daemon=True)

    def start(self) -> None:
        """Start the worker thread."""
        self._thread.start()

    def wait_for_copy(self) -> None:
        """Block until the staged copies are complete.

        Raises:
            RuntimeError: If the worker failed.
        """
        self.copy_ready.wait()
        self._reraise()

    def wait_for_update(self) -> None:
        """Block until the update is applied.

        Raises:
            RuntimeError: If the worker failed.
        """
        self.update_done.wait()
        self._thread.join()
        self._reraise()

    def done(self) -> bool:
        """Whether the update has been applied."""
        return self.update_done.is_set()

    def _reraise(self) -> None:
        if self.exception is not None:
            raise RuntimeError("Asynchronous CPU EMA update failed") from self.exception

    def _work(self) -> None:
        try:
            for item in self.items:
                if item.event is not None:
                    item.event.synchronize()
            self.copy_ready.set()
            for item in self.items:
                if item.state[EMA_INITIALIZED]:
                    source = item.tmp_cpu
                    if source.dtype != FP32:
                        if self.fp32_staging is None:
                            raise RuntimeError("CPU EMA FP32 staging buffer missing")
                        source = self.fp32_staging[: source.numel()].view(source.shape).copy_(source)
                    ema_update_(item.shadow, source, decay=self.decay)
                else:
                    item.shadow.copy_(item.tmp_cpu)
                    item.state[EMA_INITIALIZED] = True
                item.state.pop(EMA_EVENT, None)
                item.state[EMA_PENDING] = False
        except BaseException as exc:  # noqa: BLE001 - handed to the waiting thread
            self.exception = exc
            self.copy_ready.set()
        finally:
            self.update_done.set()
