"""The host side of CPU EMA: shadow updates applied by one background thread.

A due step copies every parameter into its pinned host buffer on a copy
stream; ``HostEmaWorker.submit`` then hands the batch to a single worker
thread, which waits for each copy's event and moves each float32 host shadow
to its snapshot (a lerp, or a copy for a shadow not yet initialized). One batch
is in flight at a time; its ``Future`` carries any exception of the worker, and
``wait`` re-raises it in the training thread (the reference's worker keeps the
exception and re-raises it on the next wait, ema/_cpu_job.py:104-137 of the
reference).
"""

from __future__ import annotations

from concurrent.futures import Future, ThreadPoolExecutor
from dataclasses import dataclass
from typing import Any

import torch
from torch import Tensor

from dionw_amd.ema._keys import EMA_EVENT, EMA_INITIALIZED, EMA_PENDING
from dionw_amd.ema._update import FP32, ema_update_

__all__ = ["HostEmaWorker", "HostSnapshot"]


@dataclass
class HostSnapshot:
    """One parameter's staged update.

    Attributes:
        entry: The parameter's optimizer-state entry (flags are updated in it).
        ready: Event of the copy into ``staged`` (None: already complete).
        shadow: The float32 host shadow.
        staged: The pinned host copy of the parameter.
    """

    entry: dict[str, Any]
    ready: torch.cuda.Event | None
    shadow: Tensor
    staged: Tensor

    def __post_init__(self) -> None:
        for name, tensor in (("shadow", self.shadow), ("staged snapshot", self.staged)):
            if tensor.device.type != "cpu":
                raise ValueError(f"a CPU EMA {name} must live on the CPU, got {tensor.device}")


class HostEmaWorker:
    """Applies batches of ``HostSnapshot`` on one background thread."""

    def __init__(self) -> None:
        self._pool: ThreadPoolExecutor | None = None
        self._inflight: Future[None] | None = None
        self._upcast: Tensor | None = None  # float32 scratch for 16-bit snapshots

    def submit(self, batch: list[HostSnapshot], decay: float) -> None:
        """Start applying ``batch`` (after any earlier batch has finished).

        Raises:
            RuntimeError: If the previous batch failed (re-raised here).
        """
        self.wait()
        if not batch:
            return
        need = max((s.staged.numel() for s in batch if s.staged.dtype != FP32), default=0)
        if need and (self._upcast is None or self._upcast.numel() < need):
            self._upcast = torch.empty(need, dtype=FP32)
        if self._pool is None:
            self._pool = ThreadPoolExecutor(max_workers=1, thread_name_prefix="dionw_cpu_ema")
        self._inflight = self._pool.submit(self._apply, batch, decay, self._upcast)

    def busy(self) -> bool:
        """Whether a batch is still being applied."""
        return self._inflight is not None and not self._inflight.done()

    def wait(self) -> None:
        """Block until the batch in flight (if any) is applied.

        Raises:
            RuntimeError: If the worker raised while applying it.
        """
        inflight, self._inflight = self._inflight, None
        if inflight is None:
            return
        error = inflight.exception()
        if error is not None:
            raise RuntimeError("the asynchronous CPU EMA update failed") from error

    @staticmethod
    def _apply(batch: list[HostSnapshot], decay: float, upcast: Tensor | None) -> None:
        for snap in batch:
            if snap.ready is not None:
                snap.ready.synchronize()
        for snap in batch:
            entry = snap.entry
            if not entry[EMA_INITIALIZED]:
                snap.shadow.copy_(snap.staged)
                entry[EMA_INITIALIZED] = True
            else:
                source = snap.staged
                if source.dtype != FP32:
                    if upcast is None:
                        raise RuntimeError("no float32 scratch for a 16-bit CPU EMA snapshot")
                    source = upcast[: source.numel()].view(source.shape).copy_(source)
                ema_update_(snap.shadow, source, decay=decay)
            entry.pop(EMA_EVENT, None)
            entry[EMA_PENDING] = False
