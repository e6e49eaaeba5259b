"""``OptimizerIntegratedEMA``: EMA shadows kept in ``optimizer.state[p]``.

The schedule is a pure function of the step count (``cadence_at``). A due
step updates every parameter's shadow after the optimizer's own update:

- GPU shadows: each parameter queues a copy (first update, or a restart from
  the live weights) or a lerp; ``finalize_updates`` runs each list as one
  multi-tensor HIP launch per 48 tensors. The optimizer may instead take the
  lerp inside its own pass over the new weights (``fusable_shadows``): a
  parameter it marks as fused skips the queue.
- CPU shadows: each parameter is copied into its pinned host buffer on a copy
  stream, ``HostEmaWorker`` applies the batch on a background thread, and the
  next step's stream waits for the copies on the GPU before it writes the
  parameters (no host wait; the caller's forward and backward in between run
  beside the copies). The next due step waits for the batch before reusing the
  buffers. The optimizer starts the copies of the parameters each of its
  passes writes right after that pass (``stage_written``), so they overlap the
  rest of the step; its matrix apply pass may instead write the snapshots
  itself, straight from the registers that hold the new weights
  (``stageable_buffers``, ``mark_staged``; switched by ``fuse_host_copies``).

The reference's tracker (ema/tracker.py:40-299) blocks the host on the
previous copy at every step instead; the cadence and the arithmetic (lerp with
``decay ** n``, a copy at the first update) are the same.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Final

import torch
from torch import Tensor
from torch.optim import Optimizer

from dionw_amd.ema._host_worker import HostEmaWorker, HostSnapshot
from dionw_amd.ema._keys import EMA_EVENT, EMA_INITIALIZED, EMA_PENDING, EMA_SHADOW, EMA_TMP_CPU
from dionw_amd.ema._update import FP32, foreach_ema_copy_, foreach_ema_update_
from dionw_amd.ema.config import EMAConfig, EMADevice, ProfileRegion

__all__ = ["Cadence", "OptimizerIntegratedEMA", "cadence_at"]

_STAGE_REGION: Final = "ema_stage_copy"
_FINALIZE_REGION: Final = "ema_finalize"


@dataclass(frozen=True)
class Cadence:
    """What the EMA does at one optimizer step.

    Attributes:
        update: The shadows move this step.
        from_live: Every shadow restarts as a copy of its parameter (the
            configured ``start_step``).
        decay: The lerp decay of a due update, ``decay_at_step ** n``; None
            when nothing is lerped.
    """

    update: bool
    from_live: bool
    decay: float | None


def cadence_at(config: EMAConfig, step_count: int) -> Cadence:
    """The EMA's action at optimizer step ``step_count`` (1 for the first step).

    With ``start_step = s > 0`` nothing happens before step s and step s copies
    the live weights; after it (or from the start when s = 0) an update is due
    every ``update_every_n_steps = n`` steps, lerping with the schedule's decay
    raised to n so the half-life in steps does not depend on n
    (reference tracker.py:154-175).
    """
    start, every = config.start_step, config.update_every_n_steps
    if start > 0 and step_count < start:
        return Cadence(False, False, None)
    if start > 0 and step_count == start:
        return Cadence(True, True, None)
    since = step_count - start
    if since <= 0 or since % every:
        return Cadence(False, False, None)
    return Cadence(True, False, config.decay_at_step(step_count) ** every)


def _pinned_like(param: Tensor, *, pin: bool) -> Tensor:
    """A zeroed host buffer for a parameter's snapshot (float32 and bfloat16
    kept, other dtypes staged as float32)."""
    staged = param.dtype if param.dtype in (FP32, torch.bfloat16) else FP32
    return torch.zeros(tuple(param.shape), dtype=staged, device="cpu", pin_memory=pin)


class OptimizerIntegratedEMA:
    """EMA shadows stored in an optimizer's per-parameter state.

    Attributes:
        optimizer: Owner of the per-parameter state the shadows live in.
        config: Schedule and placement.
    """

    def __init__(self, optimizer: Optimizer, config: EMAConfig,
                 profile_region: ProfileRegion) -> None:
        if config.device not in (EMADevice.GPU, EMADevice.CPU):
            raise RuntimeError(f"Unhandled EMADevice: {config.device}")
        self.optimizer = optimizer
        self.config = config
        self._region = profile_region
        self._on_gpu = config.device is EMADevice.GPU
        self._count = 0
        self._now = Cadence(False, False, None)
        self._copies: tuple[list[Tensor], list[Tensor]] = ([], [])
        self._lerps: tuple[list[Tensor], list[Tensor]] = ([], [])
        self._host = HostEmaWorker()
        self._batch: list[HostSnapshot] = []
        self._copy_streams: dict[torch.device, torch.cuda.Stream] = {}
        self._fused: set[int] = set()
        self._staged: set[int] = set()
        self._copies_unjoined = False
        # Whether the optimizer's matrix apply pass writes CPU EMA snapshots
        # itself (else they are copied on the copy stream after the pass). The
        # pass then runs at the host link's rate (~55 GB/s) on the training
        # stream, while copy-stream copies overlap whatever the caller runs
        # before the next step (its forward and backward), so it is off unless a
        # caller whose steps follow each other directly turns it on.
        self.fuse_host_copies = False

    # -- schedule --------------------------------------------------------------
    @property
    def step_count(self) -> int:
        """Optimizer steps seen by the schedule (saved with the state)."""
        return self._count

    @step_count.setter
    def step_count(self, value: int) -> None:
        if value < 0:
            raise ValueError(f"the EMA step count must be non-negative (zero or more), not {value}")
        self._count = value

    @property
    def uses_gpu_shadow(self) -> bool:
        """Whether shadows live on the parameters' GPU."""
        return self._on_gpu

    def begin_step(self) -> None:
        """Advance the schedule as an optimizer step starts."""
        if self._copies_unjoined:
            # The last due step's snapshot copies read the parameters this step
            # is about to write.
            for device, stream in self._copy_streams.items():
                torch.cuda.current_stream(device).wait_stream(stream)
            self._copies_unjoined = False
        self._fused.clear()
        self._staged.clear()
        self._count += 1
        self._now = cadence_at(self.config, self._count)
        if self._now.update and not self._on_gpu:
            self._host.wait()  # its host buffers are about to be refilled

    def should_update_this_step(self) -> bool:
        """Whether this step moves the shadows."""
        return self._now.update

    def _lerp_decay(self) -> float:
        return self.config.decay if self._now.decay is None else self._now.decay

    # -- fusion into the optimizer's own passes ----------------------------------
    def fusable_shadows(self, params: list[Tensor]) -> list[Tensor] | None:
        """The shadows of ``params`` when this step's update of every one of them
        is a GPU lerp the optimizer may take in its pass over the new weights
        (initialized float32 shadows laid out like their contiguous float32
        parameters), else None."""
        if not (self._on_gpu and self._now.update) or self._now.from_live:
            return None
        shadows = []
        for param in params:
            entry = self.optimizer.state.get(param)
            shadow = entry.get(EMA_SHADOW) if entry else None
            if (shadow is None or not entry.get(EMA_INITIALIZED, False)
                    or param.dtype is not FP32 or shadow.shape != param.shape
                    or shadow.device != param.device
                    or not (param.is_contiguous() and shadow.is_contiguous())):
                return None
            shadows.append(shadow)
        return shadows

    def fused_weight(self) -> float:
        """The lerp weight ``1 - decay`` of this step's update."""
        return 1.0 - self._lerp_decay()

    def mark_fused(self, params: list[Tensor]) -> None:
        """Record that the optimizer's pass updated these parameters' shadows."""
        self._fused.update(id(p) for p in params)

    @torch.no_grad()
    def stage_written(self, params: list[Tensor]) -> None:
        """Start the host copies of parameters the optimizer has just written
        (CPU EMA, due step): issued after the pass that wrote them, the copies
        overlap the rest of the step instead of following it."""
        if self._on_gpu or not self._now.update:
            return
        fresh = []
        for param in params:
            entry = self.optimizer.state.get(param)
            if entry is None or id(param) in self._staged:
                continue
            if EMA_SHADOW not in entry:
                self._place(param, entry, None, False)
            fresh.append((param, entry))
            self._staged.add(id(param))
        self._stage(fresh)

    def stageable_buffers(self, params: list[Tensor]) -> list[Tensor] | None:
        """The pinned host buffers the optimizer's pass over the new weights of
        ``params`` may write this step's CPU EMA snapshots into (float32,
        contiguous, laid out like their contiguous float32 CUDA parameters, not
        staged yet), else None. Parameters without a shadow get one here."""
        if self._on_gpu or not self._now.update:
            return None
        buffers = []
        for param in params:
            entry = self.optimizer.state.get(param)
            if (entry is None or id(param) in self._staged or not param.is_cuda
                    or param.dtype is not FP32 or not param.is_contiguous()):
                return None
            if EMA_SHADOW not in entry:
                self._place(param, entry, None, False)
            staged = entry[EMA_TMP_CPU]
            if (staged.dtype is not FP32 or staged.shape != param.shape
                    or not staged.is_contiguous() or not staged.is_pinned()):
                return None
            buffers.append(staged)
        return buffers

    def mark_staged(self, params: list[Tensor]) -> None:
        """Record that the work just enqueued on the current stream writes the
        snapshots of ``params`` into their host buffers (``stageable_buffers``)."""
        if not params:
            return
        ready = torch.cuda.Event()
        ready.record(torch.cuda.current_stream(params[0].device))
        for param in params:
            self._snapshot(self.optimizer.state[param], ready)
            self._staged.add(id(param))

    # -- shadows -----------------------------------------------------------------
    def _place(self, param: Tensor, entry: dict[str, Any], shadow: Tensor | None,
               initialized: bool) -> None:
        """Give ``param`` a float32 shadow on the EMA device (zeros, or a copy of
        ``shadow``) and, for CPU EMA, its pinned staging buffer."""
        if self._on_gpu and not param.is_cuda:
            raise ValueError("the EMA is configured for the GPU but a parameter is on the CPU")
        pin = self.config.pin_memory and not self._on_gpu
        device = param.device if self._on_gpu else torch.device("cpu")
        template = param if shadow is None else shadow
        fresh = torch.zeros_like(template, dtype=FP32, device=device, pin_memory=pin)
        if shadow is not None:
            fresh.copy_(shadow)
        entry[EMA_SHADOW] = fresh
        entry[EMA_INITIALIZED] = initialized
        entry[EMA_PENDING] = False
        if not self._on_gpu:
            entry[EMA_TMP_CPU] = _pinned_like(param, pin=pin)

    def restore_shadow(self, param: Tensor, saved: Tensor, initialized: bool) -> None:
        """Put a checkpoint's shadow of ``param`` on the EMA device.

        Raises:
            TypeError: If ``saved`` is not a tensor.
        """
        if not isinstance(saved, Tensor):
            raise TypeError(f"a saved {type(self.optimizer).__name__} EMA shadow is not a tensor")
        self._place(param, self.optimizer.state[param], saved, bool(initialized))

    @torch.no_grad()
    def update_param(self, param: Tensor) -> None:
        """Queue or stage one parameter's due update (parameters without
        optimizer state are skipped)."""
        with self._region(_STAGE_REGION):
            if not self._now.update or param not in self.optimizer.state:
                return
            entry = self.optimizer.state[param]
            if id(param) in self._fused:
                entry[EMA_PENDING] = False
                return
            if EMA_SHADOW not in entry:
                self._place(param, entry, None, False)
            if not self._on_gpu:
                if id(param) not in self._staged:
                    self._stage([(param, entry)])
                return
            restart = self._now.from_live or not entry[EMA_INITIALIZED]
            queue = self._copies if restart else self._lerps
            queue[0].append(entry[EMA_SHADOW])
            queue[1].append(param)
            entry[EMA_INITIALIZED] = True
            entry[EMA_PENDING] = False

    def _stage(self, items: list[tuple[Tensor, dict[str, Any]]]) -> None:
        """Copy parameters into their pinned host buffers on the copy stream,
        which first waits for the work issued so far (the writes of the
        parameters); one event per copy tells the worker when it has landed."""
        joined: set[torch.device] = set()
        for param, entry in items:
            staged = entry[EMA_TMP_CPU]
            ready = None
            if param.is_cuda and staged.is_pinned():
                stream = self._copy_streams.get(param.device)
                if stream is None:
                    stream = self._copy_streams[param.device] = torch.cuda.Stream(param.device)
                if param.device not in joined:
                    stream.wait_stream(torch.cuda.current_stream(param.device))
                    joined.add(param.device)
                with torch.cuda.stream(stream):
                    staged.copy_(param, non_blocking=True)
                    ready = torch.cuda.Event()
                    ready.record(stream)
            else:
                staged.copy_(param)
            self._snapshot(entry, ready)

    def _snapshot(self, entry: dict[str, Any], ready: torch.cuda.Event | None) -> None:
        """Queue a parameter whose host buffer is being filled (``ready`` marks
        the end of the fill) for the host worker."""
        if self._now.from_live:
            entry[EMA_INITIALIZED] = False
        entry[EMA_EVENT] = ready
        entry[EMA_PENDING] = True
        self._batch.append(HostSnapshot(entry, ready, entry[EMA_SHADOW], entry[EMA_TMP_CPU]))

    @torch.no_grad()
    def _run_device_queues(self) -> None:
        if self._copies[0]:
            foreach_ema_copy_(*self._copies)
        if self._lerps[0]:
            foreach_ema_update_(*self._lerps, decay=self._lerp_decay())
        for queue in (self._copies, self._lerps):
            queue[0].clear()
            queue[1].clear()

    @torch.no_grad()
    def finalize_updates(self) -> None:
        """Apply this step's GPU updates, or hand the staged batch to the host
        worker."""
        with self._region(_FINALIZE_REGION):
            if self._on_gpu:
                self._run_device_queues()
                self._fused.clear()
                return
            batch, self._batch = self._batch, []
            self._staged.clear()
            if not batch:
                return
            # The copies may run on beside whatever the caller enqueues until the
            # next step, which writes the parameters: that step's stream waits for
            # them first (begin_step), on the GPU.
            self._copies_unjoined = bool(self._copy_streams)
            self._host.submit(batch, self._lerp_decay())

    def flush_pending_updates(self) -> None:
        """Complete the EMA work still queued, so that the shadows can be read.

        Raises:
            RuntimeError: If the CPU worker failed.
        """
        if self._on_gpu:
            self._run_device_queues()
        else:
            self._host.wait()
