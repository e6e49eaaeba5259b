"""``OptimizerIntegratedEMA``: shadows in ``optimizer.state[p]``, GPU or CPU.

Reference: src/dionw/ema/tracker.py:40-299. GPU shadows are queued during the
step and updated at ``finalize_updates`` by the multi-tensor HIP kernels
(copies for shadows not yet initialized, lerps for the rest), with no host
synchronization; a Dion step may instead take the lerp of the parameters it
writes into its own apply and AdamW passes (``fusable_shadows``), which then
skip the queue. CPU shadows receive a snapshot copied on a side stream into
pinned buffers, then a background thread applies the update (one job in
flight at most).
"""

from __future__ import annotations

from typing import Any, Final

import torch
from torch import Tensor
from torch.optim import Optimizer

from dionw_amd.ema._cpu_job import AsyncCpuEmaItem, AsyncCpuEmaJob
from dionw_amd.ema._keys import EMA_EVENT, EMA_INITIALIZED, EMA_PENDING, EMA_SHADOW, EMA_TMP_CPU
from dionw_amd.ema._update import FP32, foreach_ema_copy_, foreach_ema_update_
from dionw_amd.ema.config import EMAConfig, EMADevice, ProfileRegion

__all__ = ["OptimizerIntegratedEMA", "new_cpu_staging"]

_STAGE_REGION: Final = "ema_stage_copy"
_FINALIZE_REGION: Final = "ema_finalize"


def new_cpu_staging(param: Tensor, *, pin: bool) -> Tensor:
    """A zero CPU buffer for a parameter's snapshot (float32 and bfloat16 kept,
    other dtypes staged as float32)."""
    dtype = param.dtype if param.dtype in (FP32, torch.bfloat16) else FP32
    return torch.zeros_like(param, dtype=dtype, device="cpu", pin_memory=pin)


class OptimizerIntegratedEMA:
    """EMA shadows stored in an optimizer's per-parameter state."""

    def __init__(self, optimizer: Optimizer, config: EMAConfig, profile_region: ProfileRegion) -> None:
        self.optimizer = optimizer
        self.config = config
        self._profile_region = profile_region
        if config.device is EMADevice.GPU:
            self._use_gpu_shadow = True
        elif config.device is EMADevice.CPU:
            self._use_gpu_shadow = False
        else:
            raise RuntimeError(f"Unhandled EMADevice: {config.device}")
        self._step_count = 0
        self._do_update = True
        self._initialize_from_live = False
        self._eff_decay: float | None = None
        self._cpu_ema_job: AsyncCpuEmaJob | None = None
        self._cpu_fp32_staging: Tensor | None = None
        self._copy_streams: dict[torch.device, torch.cuda.Stream] = {}
        self._gpu_copy: tuple[list[Tensor], list[Tensor]] = ([], [])
        self._gpu_lerp: tuple[list[Tensor], list[Tensor]] = ([], [])
        # Parameters whose update of this step the optimizer's own pass took.
        self._fused: set[int] = set()

    # -- schedule ------------------------------------------------------------
    @property
    def step_count(self) -> int:
        """Optimizer steps seen by the schedule (saved with the state)."""
        return self._step_count

    @step_count.setter
    def step_count(self, value: int) -> None:
        if value < 0:
            raise ValueError(f"EMA step_count must be non-negative, got {value}")
        self._step_count = value

    @property
    def uses_gpu_shadow(self) -> bool:
        """Whether shadows live on the parameters' GPU."""
        return self._use_gpu_shadow

    def begin_step(self) -> None:
        """Advance the schedule at the start of an optimizer step."""
        self._fused.clear()
        if not self._use_gpu_shadow:
            self._wait_for_previous_snapshot_copy()
        self._step_count += 1
        n = self.config.update_every_n_steps
        start = self.config.start_step
        self._initialize_from_live = start > 0 and self._step_count == start
        if start > 0 and self._step_count < start:
            self._do_update = False
        elif self._initialize_from_live:
            self._do_update = True
        else:
            since = self._step_count - start
            self._do_update = since > 0 and since % n == 0
        decay = self.config.decay_at_step(self._step_count)
        due_lerp = self._do_update and not self._initialize_from_live
        self._eff_decay = decay**n if due_lerp else None
        if self._do_update and not self._use_gpu_shadow:
            self._wait_for_previous_cpu_update()

    def should_update_this_step(self) -> bool:
        """Whether this step updates the shadows."""
        return self._do_update

    # -- fusion into the optimizer's passes ------------------------------------
    def fusable_shadows(self, params: list[Tensor]) -> list[Tensor] | None:
        """The shadows of ``params`` if this step's update of every one of them
        is a GPU lerp that the optimizer may apply in its own pass over the new
        weights (initialized float32 shadows laid out like their contiguous
        float32 parameters), else None."""
        if not (self._use_gpu_shadow and self._do_update) or self._initialize_from_live:
            return None
        shadows = []
        for param in params:
            state = self.optimizer.state.get(param)
            shadow = state.get(EMA_SHADOW) if state else None
            if (
                shadow is None
                or not state.get(EMA_INITIALIZED, False)
                or param.dtype != FP32
                or shadow.shape != param.shape
                or shadow.device != param.device
                or not (param.is_contiguous() and shadow.is_contiguous())
            ):
                return None
            shadows.append(shadow)
        return shadows

    def fused_weight(self) -> float:
        """The lerp weight of this step's update (as foreach_ema_update_ forms it)."""
        decay = self.config.decay if self._eff_decay is None else self._eff_decay
        return 1.0 - decay

    def mark_fused(self, params: list[Tensor]) -> None:
        """Record that the optimizer's pass updated these parameters' shadows."""
        self._fused.update(id(param) for param in params)

    # -- queueing ------------------------------------------------------------
    def _create_shadow(self, param: Tensor, state: dict[str, Any]) -> None:
        if self._use_gpu_shadow and not param.is_cuda:
            raise ValueError("EMA configured for the GPU but a parameter is on the CPU")
        pin = self.config.pin_memory and not self._use_gpu_shadow
        device = param.device if self._use_gpu_shadow else torch.device("cpu")
        state[EMA_SHADOW] = torch.zeros_like(param, dtype=FP32, device=device, pin_memory=pin)
        state[EMA_INITIALIZED] = False
        if not self._use_gpu_shadow:
            state[EMA_TMP_CPU] = new_cpu_staging(param, pin=pin)

    @torch.no_grad()
    def update_param(self, param: Tensor) -> None:
        """Stage one parameter's update (parameters without state are skipped)."""
        with self._profile_region(_STAGE_REGION):
            if not self._do_update or param not in self.optimizer.state:
                return
            state = self.optimizer.state[param]
            if id(param) in self._fused:
                state[EMA_PENDING] = False
                return
            if EMA_SHADOW not in state:
                self._create_shadow(param, state)
            if self._use_gpu_shadow:
                if self._initialize_from_live or not state[EMA_INITIALIZED]:
                    self._gpu_copy[0].append(state[EMA_SHADOW])
                    self._gpu_copy[1].append(param)
                    state[EMA_INITIALIZED] = True
                else:
                    self._gpu_lerp[0].append(state[EMA_SHADOW])
                    self._gpu_lerp[1].append(param)
                state[EMA_PENDING] = False
            else:
                self._stage_cpu_snapshot(param, state)

    def _copy_stream_for(self, device: torch.device) -> torch.cuda.Stream:
        stream = self._copy_streams.get(device)
        if stream is None:
            stream = self._copy_streams[device] = torch.cuda.Stream(device=device)
        return stream

    def _stage_cpu_snapshot(self, param: Tensor, state: dict[str, Any]) -> None:
        if self._initialize_from_live:
            state[EMA_INITIALIZED] = False
        tmp_cpu = state[EMA_TMP_CPU]
        event = None
        if param.is_cuda and tmp_cpu.is_pinned():
            side = self._copy_stream_for(param.device)
            side.wait_stream(torch.cuda.current_stream(param.device))
            with torch.cuda.stream(side):
                tmp_cpu.copy_(param, non_blocking=True)
                event = torch.cuda.Event(blocking=False)
                event.record(side)
        else:
            tmp_cpu.copy_(param, non_blocking=False)
        state[EMA_EVENT] = event
        state[EMA_PENDING] = True

    # -- applying ------------------------------------------------------------
    @torch.no_grad()
    def _finalize_gpu_updates(self) -> None:
        if self._gpu_copy[0]:
            foreach_ema_copy_(*self._gpu_copy)
            self._gpu_copy[0].clear()
            self._gpu_copy[1].clear()
        if self._gpu_lerp[0]:
            decay = self.config.decay if self._eff_decay is None else self._eff_decay
            foreach_ema_update_(*self._gpu_lerp, decay=decay)
            self._gpu_lerp[0].clear()
            self._gpu_lerp[1].clear()

    @torch.no_grad()
    def finalize_updates(self) -> None:
        """Apply this step's GPU updates, or start the CPU worker on them."""
        with self._profile_region(_FINALIZE_REGION):
            if self._use_gpu_shadow:
                self._finalize_gpu_updates()
                self._fused.clear()
                return
            if not self._do_update:
                return
            decay = self.config.decay if self._eff_decay is None else self._eff_decay
            items = []
            for group in self.optimizer.param_groups:
                for param in group["params"]:
                    state = self.optimizer.state.get(param)
                    if state and state.get(EMA_PENDING, False):
                        items.append(
                            AsyncCpuEmaItem(state, state[EMA_EVENT], state[EMA_SHADOW],
                                            state[EMA_TMP_CPU])
                        )
            if not items:
                return
            if self._cpu_ema_job is not None:
                raise RuntimeError("CPU EMA job already pending after the pre-step wait")
            job = AsyncCpuEmaJob(items=items, decay=decay, fp32_staging=self._staging_for(items))
            self._cpu_ema_job = job
            job.start()

    def _staging_for(self, items: list[AsyncCpuEmaItem]) -> Tensor | None:
        need = max((i.tmp_cpu.numel() for i in items if i.tmp_cpu.dtype != FP32), default=0)
        if need == 0:
            return None
        if self._cpu_fp32_staging is None or self._cpu_fp32_staging.numel() < need:
            self._cpu_fp32_staging = torch.empty(need, dtype=FP32, device="cpu")
        return self._cpu_fp32_staging

    # -- waiting ---------------------------------------------------------------
    def _wait_for_previous_snapshot_copy(self) -> None:
        job = self._cpu_ema_job
        if job is None:
            return
        job.wait_for_copy()
        if job.done():
            job.wait_for_update()
            self._cpu_ema_job = None

    def _wait_for_previous_cpu_update(self) -> None:
        job = self._cpu_ema_job
        if job is not None:
            job.wait_for_update()
            self._cpu_ema_job = None

    def flush_pending_updates(self) -> None:
        """Finish queued EMA work before the shadows are read.

        Raises:
            RuntimeError: If the CPU worker failed.
        """
        if self._use_gpu_shadow:
            self._finalize_gpu_updates()
        else:
            self._wait_for_previous_cpu_update()
