"""``Dion``: row-selected NorMuon on matrices, AdamW on the rest, one learning rate.

A step runs, on the current HIP stream and without waiting on the host:

1. every matrix bucket in runs — maximal stretches of consecutive parameters
   with gradients, each at most ``MAX_RUN_ELEMENTS`` update elements (a larger
   parameter runs alone) — through ``step_run``: momentum, row selection,
   the orthogonalization, NorMuon and the weight update (decoupled decay on
   every row), as a handful of HIP launches per run. Inside a step the runs
   queue after their momentum passes and their Newton-Schulz products go out
   together in grouped launches;
2. every AdamW group through one multi-tensor launch per 48 tensors;
3. the due EMA update (``IntegratedEMAOptimizer``), fused into the passes of
   step 1 and 2 where it can be.

``step_run`` and ``MAX_RUN_ELEMENTS`` are read from this module at each step,
so callers may patch them (reference optimizer.py:324-369). Matrix state is
packed into buckets at the first step after the groups or the state change.
"""

from __future__ import annotations

from collections.abc import Callable, Iterable, Iterator
from contextlib import contextmanager
from contextvars import ContextVar
from typing import Any, TypeVar

import torch
from torch import Tensor

from dionw_amd import _workspace
from dionw_amd._adamw import adamw_step, init_adamw_state
from dionw_amd._buckets import Bucket, pack_buckets
from dionw_amd._groups import GroupSpec, check_decays, check_parameter, refuse_structural_change
from dionw_amd._keys import (
    EXP_AVG_STATE,
    FRACTION_KEY,
    MOMENTUM_FORM_KEY,
    MOMENTUM_KEY,
    MUON_BETA2_KEY,
    NEWTON_SCHULZ_KEY,
    NUM_HEADS_KEY,
    ROUTE_KEY,
    ROW_NORMALIZATION_KEY,
)
from dionw_amd._matrix_step import (
    ACTIVE_RUNS,
    MAX_RUN_ELEMENTS,
    PROFILE_REGION,
    RunQueue,
    step_run,
)
from dionw_amd.ema import EMAConfig, IntegratedEMAOptimizer, ProfileRegion, no_profile
from dionw_amd.ema._fusion import ACTIVE_EMA
from dionw_amd.matrix_update import DION3_UPDATE, MatrixUpdate
from dionw_amd.routing import RouteKind

__all__ = ["ADAMW_REGION", "MAX_RUN_ELEMENTS", "NEWTON_SCHULZ_KEY", "Dion", "step_run"]

# The named region around a step's AdamW groups (the matrix stages name theirs
# in _matrix_step; the EMA's are the tracker's).
ADAMW_REGION = "adamw"

_T = TypeVar("_T")


@contextmanager
def _bound(var: ContextVar[_T], value: _T) -> Iterator[None]:
    token = var.set(value)
    try:
        yield
    finally:
        var.reset(token)


def _runs(bucket: Bucket) -> Iterator[list[int]]:
    """The bucket's runs: positions of consecutive parameters with gradients,
    split so that no run exceeds ``MAX_RUN_ELEMENTS`` update elements."""
    cap = MAX_RUN_ELEMENTS
    per_block = bucket.selected_rows * bucket.cols
    run: list[int] = []
    size = 0
    for position, param in enumerate(bucket.params):
        if param.grad is None:
            if run:
                yield run
            run, size = [], 0
            continue
        elements = (bucket.offsets[position + 1] - bucket.offsets[position]) * per_block
        if run and size + elements > cap:
            yield run
            run, size = [], 0
        run.append(position)
        size += elements
    if run:
        yield run


class Dion(IntegratedEMAOptimizer):
    """Dion on matrices and AdamW on the rest, with an optional integrated EMA.

    Build the groups with ``param_groups(model)``; ``lr`` is an
    AdamW-equivalent learning rate for every parameter.
    """

    def __init__(
        self,
        params: Iterable[dict[str, Any]],
        *,
        lr: float,
        momentum: float = 0.95,
        muon_beta2: float = 0.95,
        betas: tuple[float, float] = (0.9, 0.95),
        weight_decay: float = 0.0,
        eps: float = 1e-8,
        matrix_update: MatrixUpdate = DION3_UPDATE,
        ema: EMAConfig | None = None,
        profile_region: ProfileRegion = no_profile,
    ) -> None:
        """Create the optimizer.

        Raises:
            TypeError: For a group without a route, or parameters that are not float32.
            ValueError: For out-of-range hyperparameters, Nesterov momentum with
                row selection, or parameters off the GPU.
        """
        check_decays(lr=lr, weight_decay=weight_decay, eps=eps,
                     decays={MOMENTUM_KEY: momentum, MUON_BETA2_KEY: muon_beta2,
                             "beta1": betas[0], "beta2": betas[1]})
        self._packed: list[Bucket] | None = None
        super().__init__(params, {
            "lr": lr,
            "betas": betas,
            "eps": eps,
            "weight_decay": weight_decay,
            MOMENTUM_KEY: momentum,
            MUON_BETA2_KEY: muon_beta2,
            FRACTION_KEY: 1.0,
            NUM_HEADS_KEY: None,
            NEWTON_SCHULZ_KEY: matrix_update.newton_schulz.value,
            ROW_NORMALIZATION_KEY: matrix_update.row_normalization.value,
            MOMENTUM_FORM_KEY: matrix_update.momentum_form.value,
        })
        self._profile_region = profile_region
        self._init_integrated_ema(ema, profile_region)

    # -- groups and state ------------------------------------------------------
    def _repack(self) -> None:
        """Drop the packed buckets (and the step's scratch buffers, sized for
        them): the next step packs the state again."""
        self._packed = None
        _workspace.release()

    def add_param_group(self, param_group: dict[str, Any]) -> None:
        """Check and add a group; AdamW state is created now, matrix state is
        repacked at the next step.

        Raises:
            TypeError: Without a route, for a set of params or non-float32 ones.
            ValueError: For an invalid route, option or fraction, or a
                parameter off the GPU.
        """
        given = param_group["params"]
        if isinstance(given, set):
            raise TypeError("a Dion param group lists its params in order (a list or tuple), not as a set")
        params = [given] if isinstance(given, Tensor) else list(given)
        for param in params:
            check_parameter(param)
        group = {**param_group, "params": params}
        spec = GroupSpec.of({**self.defaults, **group})
        super().add_param_group(group)
        self._repack()
        # With AdamW state present from the start, an integrated EMA tracks
        # every parameter; matrix state appears with the buckets.
        if spec.kind is RouteKind.ADAMW:
            for param in params:
                init_adamw_state(param, self.state[param])

    def initialize_state(self, param: Tensor) -> None:
        """Create a parameter's state before its first step, without updating it.

        Raises:
            ValueError: For a parameter that no group of this optimizer holds (not in the optimizer).
        """
        owner = next((g for g in self.param_groups if any(p is param for p in g["params"])),
                     None)
        if owner is None:
            raise ValueError("the parameter is not in the optimizer")
        if GroupSpec.of(owner).kind is RouteKind.MATRIX:
            self._buckets()
        elif EXP_AVG_STATE not in self.state[param]:
            init_adamw_state(param, self.state[param])

    def load_state_dict(self, state_dict: dict[str, Any]) -> None:
        """Load a checkpoint of the same group structure; matrix state is
        repacked at the next step.

        Raises:
            ValueError: If the saved groups differ in number or in a structural
                key (route, fraction, heads, update options).
        """
        groups = refuse_structural_change(state_dict["param_groups"], self.param_groups)
        super().load_state_dict({**state_dict, "param_groups": groups})
        self._repack()

    def _buckets(self) -> list[Bucket]:
        if self._packed is None:
            self._packed = pack_buckets(self.param_groups, self.state)
        return self._packed

    def _check_capturable(self) -> None:
        """Refuse a step under HIP graph capture that a replay would not repeat.

        A captured step replays the launches of the step it recorded: its
        gradient tensors, hyperparameters and step sizes. Two things a step
        can do are not launches and must not be recorded: packing the matrix
        state (zeroed buckets and copies of earlier state, after construction,
        ``add_param_group`` or ``load_state_dict``), which a replay would redo
        on every step, and the EMA's host-side schedule.

        Raises:
            RuntimeError: If the state is not packed or an EMA is attached.
        """
        if self._packed is None:
            raise RuntimeError(
                "Dion.step under graph capture: the matrix state is not packed (the first step "
                "after construction, add_param_group or load_state_dict packs it); run one "
                "eager step first, or call initialize_state on a matrix parameter")
        if self.ema is not None:
            raise RuntimeError("Dion.step under graph capture: the EMA's schedule runs on the "
                               "host each step and cannot be replayed; capture without an EMA")

    # -- the step ----------------------------------------------------------------
    @torch.no_grad()
    def step(self, closure: Callable[[], float] | None = None) -> float | None:  # type: ignore[override]
        """Update every parameter with a gradient; then the due EMA update.

        Raises:
            RuntimeError: If the EMA weights are in the parameters.
        """
        if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
            self._check_capturable()
        with self._ema_cadence():
            loss = None
            if closure is not None:
                with torch.enable_grad():
                    loss = closure()
            queue = RunQueue()
            region = self._profile_region
            with (_bound(ACTIVE_EMA, self.ema), _bound(ACTIVE_RUNS, queue),
                  _bound(PROFILE_REGION, region)):
                for bucket in self._buckets():
                    group = self.param_groups[bucket.group_index]
                    for positions in _runs(bucket):
                        step_run(bucket, positions, group, self.state)
                queue.flush()
                adamw_groups = [g for g in self.param_groups
                                if g[ROUTE_KEY] == RouteKind.ADAMW.value]
                if adamw_groups:
                    with region(ADAMW_REGION):
                        for group in adamw_groups:
                            adamw_step(group, self.state)
        return loss

