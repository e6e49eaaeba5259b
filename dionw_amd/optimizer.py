"""``Dion``: row-selected NorMuon on matrices, AdamW on the rest, one LR.

Reference: src/dionw/optimizer.py:1-424. Per matrix block: ``M += G``; keep
the top ``k = ceil(fraction * rows)`` rows by momentum l1 norm and decay them
(error feedback); orthogonalize them (Newton-Schulz, five steps); NorMuon row
normalization; ``W[rows] -= lr * 0.2 * sqrt(max(rows, cols)) * c * O`` with
``c = sqrt(min(rows, cols) / min(k, cols))``; decoupled weight decay ``W *= 1 -
lr * weight_decay`` on every row. Other parameters get AdamW. Every stage is a
HIP kernel launched on the current stream; a step never synchronizes with the
host (except CPU EMA's waits).
"""

from __future__ import annotations

from collections.abc import Callable, Iterable
from typing import Any

import torch
from torch import Tensor
from torch.optim import Optimizer

from dionw_amd._adamw import adamw_step, init_adamw_state
from dionw_amd._buckets import Bucket, block_shape, build_buckets
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
    STRUCTURAL_KEYS,
)
from dionw_amd._matrix_step import (
    ACTIVE_RUNS,
    MAX_RUN_ELEMENTS,
    RunQueue,
    run_elements,
    step_run,
)
from dionw_amd.ema._fusion import ACTIVE_EMA
from dionw_amd.ema import EMAConfig, IntegratedEMAOptimizer, ProfileRegion, no_profile
from dionw_amd.matrix_update import DION3_UPDATE, MatrixUpdate, MomentumForm, RowNormalization
from dionw_amd.newton_schulz import NewtonSchulz
from dionw_amd.routing import RouteKind

__all__ = ["MAX_RUN_ELEMENTS", "NEWTON_SCHULZ_KEY", "Dion", "step_run"]


def _check_hyperparameters(lr: float, weight_decay: float, eps: float, coefficients: dict[str, float]) -> None:
    if lr < 0.0 or weight_decay < 0.0 or eps <= 0.0:
        raise ValueError("lr and weight_decay must be >= 0 and eps > 0")
    for name, value in coefficients.items():
        if not 0.0 <= value < 1.0:
            raise ValueError(f"{name} must be in [0, 1), got {value}")


def _check_group(group: dict[str, Any]) -> None:
    if ROUTE_KEY not in group:
        raise TypeError(
            "Dion param groups need a route: build them with "
            "dionw.param_groups(model) instead of passing parameters directly"
        )
    NewtonSchulz(group[NEWTON_SCHULZ_KEY])
    RowNormalization(group[ROW_NORMALIZATION_KEY])
    MomentumForm(group[MOMENTUM_FORM_KEY])
    if float(group["lr"]) < 0.0 or float(group["weight_decay"]) < 0.0:
        raise ValueError("a group's lr and weight_decay must be >= 0")
    kind = RouteKind(group[ROUTE_KEY])
    if kind is RouteKind.ADAMW:
        return
    if kind is not RouteKind.MATRIX:
        raise RuntimeError(f"Unhandled RouteKind: {kind}")
    fraction = float(group[FRACTION_KEY])
    if not 0.0 < fraction <= 1.0:
        raise ValueError(f"fraction must be in (0, 1], got {fraction}")
    if MomentumForm(group[MOMENTUM_FORM_KEY]) is MomentumForm.NESTEROV and fraction < 1.0:
        raise ValueError(
            f"Nesterov momentum needs every row per step, got fraction {fraction}: "
            "build the groups with fraction=1.0 or use MomentumForm.HEAVY_BALL"
        )
    for param in group["params"]:
        if param.ndim < 2:
            raise ValueError(f"a matrix group holds a {param.ndim}-D parameter; route it to AdamW")
        block_shape(param, group[NUM_HEADS_KEY])


def _check_param(param: Tensor) -> None:
    if not param.is_cuda:
        raise ValueError(f"Dion runs on CUDA devices, got a parameter on {param.device}")
    if param.dtype != torch.float32:
        raise TypeError(
            f"Dion needs float32 parameters, got {param.dtype}: keep float32 master "
            "weights and run the forward and backward in bfloat16 (autocast)"
        )


def _with_pre_option_keys(saved: list[dict[str, Any]]) -> list[dict[str, Any]]:
    """Saved groups from before the row-normalization / momentum-form options
    had the only update of the time (NorMuon, heavy ball)."""
    legacy = {
        ROW_NORMALIZATION_KEY: RowNormalization.NORMUON.value,
        MOMENTUM_FORM_KEY: MomentumForm.HEAVY_BALL.value,
    }
    return [{**legacy, **group} if ROUTE_KEY in group else group for group in saved]


def _check_structure(saved: list[dict[str, Any]], current: list[dict[str, Any]]) -> None:
    if len(saved) != len(current):
        raise ValueError(f"Dion state has {len(saved)} param groups, the optimizer {len(current)}")
    for index, (old, new) in enumerate(zip(saved, current, strict=True)):
        for key in STRUCTURAL_KEYS:
            if key not in old:
                raise ValueError(
                    f"Dion state group {index} has no {key!r}: it was not saved by dionw.Dion"
                )
            if old[key] != new[key]:
                raise ValueError(
                    f"Dion state group {index} {key!r}: checkpoint={old[key]!r}, "
                    f"optimizer={new[key]!r}. Build the groups as the checkpoint was built "
                    "to resume it."
                )


class _DionCore(Optimizer):
    """The Dion and AdamW updates over routed param groups (no EMA)."""

    def __init__(
        self,
        params: Iterable[dict[str, Any]],
        *,
        lr: float,
        momentum: float,
        muon_beta2: float,
        betas: tuple[float, float],
        weight_decay: float,
        eps: float,
        matrix_update: MatrixUpdate,
    ) -> None:
        _check_hyperparameters(
            lr,
            weight_decay,
            eps,
            {MOMENTUM_KEY: momentum, MUON_BETA2_KEY: muon_beta2, "beta1": betas[0],
             "beta2": betas[1]},
        )
        defaults = {
            "lr": lr,
            MOMENTUM_KEY: momentum,
            MUON_BETA2_KEY: muon_beta2,
            "betas": betas,
            "weight_decay": weight_decay,
            "eps": eps,
            FRACTION_KEY: 1.0,
            NUM_HEADS_KEY: None,
            NEWTON_SCHULZ_KEY: matrix_update.newton_schulz.value,
            ROW_NORMALIZATION_KEY: matrix_update.row_normalization.value,
            MOMENTUM_FORM_KEY: matrix_update.momentum_form.value,
        }
        self._buckets: list[Bucket] | None = None
        super().__init__(params, defaults)

    def add_param_group(self, param_group: dict[str, Any]) -> None:
        """Validate and add a group; matrix state is repacked on the next step.

        Raises:
            TypeError: Without a route, for a set of params, or non-float32 ones.
            ValueError: For an invalid route, kind or fraction, or a parameter
                off the GPU.
        """
        params = param_group["params"]
        if isinstance(params, set):
            raise TypeError("Dion param group params must be ordered, not a set")
        group = {**param_group, "params": [params] if isinstance(params, Tensor) else list(params)}
        for param in group["params"]:
            _check_param(param)
        _check_group({**self.defaults, **group})
        super().add_param_group(group)
        self._buckets = None
        # AdamW state exists from the start, so an integrated EMA tracks every
        # parameter; matrix state exists from the first step (the buckets).
        if RouteKind(group[ROUTE_KEY]) is RouteKind.ADAMW:
            for param in group["params"]:
                init_adamw_state(param, self.state[param])

    def initialize_state(self, param: Tensor) -> None:
        """Create a parameter's state before its first step, without an update.

        Raises:
            ValueError: If ``param`` is not in the optimizer.
        """
        group = next((g for g in self.param_groups if any(p is param for p in g["params"])), None)
        if group is None:
            raise ValueError("parameter is not in the optimizer")
        kind = RouteKind(group[ROUTE_KEY])
        if kind is RouteKind.MATRIX:
            self._ensure_buckets()
        elif kind is RouteKind.ADAMW:
            if EXP_AVG_STATE not in self.state[param]:
                init_adamw_state(param, self.state[param])
        else:
            raise RuntimeError(f"Unhandled RouteKind: {kind}")

    def load_state_dict(self, state_dict: dict[str, Any]) -> None:
        """Load, then repack matrix state into buckets on the next step.

        Raises:
            ValueError: If the saved groups differ in count or structural keys.
        """
        saved = _with_pre_option_keys(state_dict["param_groups"])
        _check_structure(saved, self.param_groups)
        super().load_state_dict({**state_dict, "param_groups": saved})
        self._buckets = None

    @torch.no_grad()
    def step(self, closure: Callable[[], float] | None = None) -> float | None:  # type: ignore[override]
        """Update every parameter with a gradient (matrix buckets, then AdamW)."""
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        # A due GPU EMA update can ride on the passes that write the new weights.
        token = ACTIVE_EMA.set(getattr(self, "ema", None))
        # Bucket runs queue after their momentum passes; their Newton-Schulz
        # calls then run as grouped launches.
        queue = RunQueue()
        runs_token = ACTIVE_RUNS.set(queue)
        try:
            for bucket in self._ensure_buckets():
                self._step_bucket(bucket)
            queue.flush()
            for group in self.param_groups:
                if RouteKind(group[ROUTE_KEY]) is RouteKind.ADAMW:
                    adamw_step(group, self.state)
        finally:
            ACTIVE_RUNS.reset(runs_token)
            ACTIVE_EMA.reset(token)
        return loss

    def _ensure_buckets(self) -> list[Bucket]:
        if self._buckets is None:
            self._buckets = build_buckets(self.param_groups, self.state)
        return self._buckets

    def _step_bucket(self, bucket: Bucket) -> None:
        """Step the bucket's parameters with gradients in contiguous runs of at
        most ``MAX_RUN_ELEMENTS`` update elements (a larger parameter runs alone)."""
        group = self.param_groups[bucket.group_index]
        run: list[int] = []
        elements = 0
        for position, param in enumerate(bucket.params):
            size = run_elements(bucket, position)
            if run and (param.grad is None or elements + size > MAX_RUN_ELEMENTS):
                step_run(bucket, run, group, self.state)
                run, elements = [], 0
            if param.grad is not None:
                run.append(position)
                elements += size
        if run:
            step_run(bucket, run, group, self.state)


class Dion(IntegratedEMAOptimizer, _DionCore):
    """Dion on matrices, AdamW on the rest, with an optional integrated EMA.

    Build the groups with ``param_groups(model)``. ``lr`` is an
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
            TypeError: For groups without a route or non-float32 parameters.
            ValueError: For out-of-range hyperparameters, Nesterov momentum with
                row selection, or parameters off the GPU.
        """
        super().__init__(
            params,
            lr=lr,
            momentum=momentum,
            muon_beta2=muon_beta2,
            betas=betas,
            weight_decay=weight_decay,
            eps=eps,
            matrix_update=matrix_update,
        )
        self._init_integrated_ema(ema, profile_region)
