"""What a Dion param group means, read once into a typed record.

A group dict carries torch's keys (``params``, ``lr``, ``betas``, ``eps``,
``weight_decay``) and Dion's (route, row fraction, head split, the three
options of the matrix update, the momentum and NorMuon decays; their names are
the checkpoint contract in ``_keys``). ``GroupSpec.of`` turns a merged group
(defaults under the user's entries) into a frozen record and raises on
anything the step could not run. The structural part of a group — route,
fraction, heads and the update options — is fixed for the life of its state:
``refuse_structural_change`` compares it between a checkpoint and the live
groups, because torch would otherwise restore the checkpoint's values silently.

Error types and the message fragments callers match follow the reference
(optimizer.py:81-316): TypeError mentioning ``dionw.param_groups`` for a group
without a route and "float32 parameters" for other dtypes; ValueError
mentioning "CUDA", "fraction", "momentum", "does not divide", "route it to
AdamW", "lr and weight_decay", "Nesterov momentum needs every row", and the
quoted name of a structural key that differs.
"""

from __future__ import annotations

from collections.abc import Mapping, Sequence
from dataclasses import dataclass
from typing import Any, Final

import torch
from torch import Tensor

from dionw_amd._keys import (
    FRACTION_KEY,
    MOMENTUM_FORM_KEY,
    NEWTON_SCHULZ_KEY,
    NUM_HEADS_KEY,
    ROUTE_KEY,
    ROW_NORMALIZATION_KEY,
    STRUCTURAL_KEYS,
)
from dionw_amd.matrix_update import MomentumForm, RowNormalization
from dionw_amd.newton_schulz import NewtonSchulz
from dionw_amd.routing import RouteKind

__all__ = [
    "GroupSpec",
    "check_decays",
    "check_parameter",
    "matrix_blocks",
    "refuse_structural_change",
]

# Checkpoints written before the row-normalization and momentum-form options
# existed ran the only update of the time: NorMuon with heavy-ball momentum.
_BEFORE_OPTIONS: Final[dict[str, str]] = {
    ROW_NORMALIZATION_KEY: RowNormalization.NORMUON.value,
    MOMENTUM_FORM_KEY: MomentumForm.HEAVY_BALL.value,
}


def matrix_blocks(param: Tensor, num_heads: int | None) -> tuple[int, int, int]:
    """``(blocks, rows, cols)`` of a matrix parameter: trailing dims flatten into
    columns and a head split divides the rows into ``num_heads`` blocks.

    Raises:
        ValueError: For a head count that leaves a remainder of rows.
    """
    rows = int(param.shape[0])
    cols = int(param.shape[1:].numel())  # trailing dims flattened
    heads = 1 if num_heads is None else num_heads
    if rows % heads:
        raise ValueError(f"{heads} heads: the count does not divide the {rows} rows")
    return heads, rows // heads, cols


def check_decays(*, lr: float, weight_decay: float, eps: float,
                 decays: Mapping[str, float]) -> None:
    """The optimizer-wide hyperparameters: ``lr, weight_decay >= 0``, ``eps > 0``
    and every decay (momentum, NorMuon beta2, AdamW betas) in [0, 1).

    Raises:
        ValueError: Naming the first value out of range.
    """
    if not (lr >= 0.0 and weight_decay >= 0.0 and eps > 0.0):
        raise ValueError("lr and weight_decay must be >= 0 and eps > 0, got "
                         f"lr={lr}, weight_decay={weight_decay}, eps={eps}")
    bad = [(name, v) for name, v in decays.items() if not 0.0 <= v < 1.0]
    if bad:
        name, value = bad[0]
        raise ValueError(f"{name} = {value} lies outside [0, 1)")


def check_parameter(param: Tensor) -> None:
    """A parameter the HIP kernels can update: on a GPU, float32.

    Raises:
        ValueError: For a parameter off the GPU (``is_cuda`` holds for HIP
            devices under PyTorch-ROCm).
        TypeError: For other dtypes than float32.
    """
    if not param.is_cuda:
        raise ValueError(f"Dion updates parameters on CUDA (HIP) devices, got one on "
                         f"{param.device}")
    if param.dtype is not torch.float32:
        raise TypeError(f"Dion keeps float32 parameters, got {param.dtype}: hold float32 "
                        "master weights and run forward and backward under autocast")


@dataclass(frozen=True)
class GroupSpec:
    """The meaning of one param group.

    Attributes:
        kind: MATRIX (Dion) or ADAMW.
        fraction: Share of each block's rows updated per step (MATRIX).
        num_heads: Row split of each parameter, or None (MATRIX).
        newton_schulz: The orthogonalization.
        row_normalization: NorMuon or none.
        momentum_form: Heavy ball or Nesterov.
    """

    kind: RouteKind
    fraction: float
    num_heads: int | None
    newton_schulz: NewtonSchulz
    row_normalization: RowNormalization
    momentum_form: MomentumForm

    @classmethod
    def of(cls, group: Mapping[str, Any]) -> GroupSpec:
        """Read (and check) a group with the optimizer's defaults merged in.

        Raises:
            TypeError: Without a route.
            ValueError: For an unknown option value, a negative lr or weight
                decay, a fraction outside (0, 1], Nesterov momentum with row
                selection, or a matrix parameter that cannot be blocked.
        """
        if ROUTE_KEY not in group:
            raise TypeError("a Dion param group needs a route: build the groups with "
                            "dionw.param_groups(model) rather than passing parameters")
        if not (float(group["lr"]) >= 0.0 and float(group["weight_decay"]) >= 0.0):
            raise ValueError("a group's lr and weight_decay must be >= 0, got "
                             f"lr={group['lr']}, weight_decay={group['weight_decay']}")
        spec = cls(
            kind=RouteKind(group[ROUTE_KEY]),
            fraction=float(group[FRACTION_KEY]),
            num_heads=group[NUM_HEADS_KEY],
            newton_schulz=NewtonSchulz(group[NEWTON_SCHULZ_KEY]),
            row_normalization=RowNormalization(group[ROW_NORMALIZATION_KEY]),
            momentum_form=MomentumForm(group[MOMENTUM_FORM_KEY]),
        )
        if spec.kind is RouteKind.MATRIX:
            spec._check_matrix(group["params"])
        elif spec.kind is not RouteKind.ADAMW:
            raise RuntimeError(f"Unhandled RouteKind: {spec.kind}")
        return spec

    def _check_matrix(self, params: Sequence[Tensor]) -> None:
        if not 0.0 < self.fraction <= 1.0:
            raise ValueError(f"the row fraction {self.fraction} lies outside (0, 1]")
        if self.momentum_form is MomentumForm.NESTEROV and self.fraction < 1.0:
            raise ValueError(
                f"Nesterov momentum needs every row per step (fraction 1.0), got fraction "
                f"{self.fraction}: use MomentumForm.HEAVY_BALL with row selection")
        for param in params:
            if param.ndim < 2:
                raise ValueError(f"a {param.ndim}-D parameter cannot take the matrix update; "
                                 "route it to AdamW")
            matrix_blocks(param, self.num_heads)


def refuse_structural_change(saved: Sequence[Mapping[str, Any]],
                             live: Sequence[Mapping[str, Any]]) -> list[dict[str, Any]]:
    """The saved groups, completed for checkpoints from before the update
    options, after checking that each matches its live group structurally.

    Raises:
        ValueError: For a different number of groups, or a structural key that
            is missing from the checkpoint or differs (its name quoted).
    """
    if len(saved) != len(live):
        raise ValueError(f"the Dion state has {len(saved)} param groups, the optimizer "
                         f"{len(live)}")
    completed = [{**_BEFORE_OPTIONS, **g} if ROUTE_KEY in g else dict(g) for g in saved]
    for index, (old, new) in enumerate(zip(completed, live)):
        for key in STRUCTURAL_KEYS:
            if key not in old:
                raise ValueError(f"param group {index} of the Dion state has no {key!r}: it was "
                                 "not written by a Dion optimizer")
            if old[key] != new[key]:
                raise ValueError(
                    f"param group {index} {key!r} differs: checkpoint {old[key]!r}, optimizer "
                    f"{new[key]!r}; build the groups as they were built for the checkpoint")
    return completed
