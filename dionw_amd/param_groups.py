"""``param_groups(model)``: route every parameter and build Dion param groups.

Reference: src/dionw/param_groups.py:89-270. A declared route wins (a
``RouteProvider`` module's ``dion_routes`` or the ``routes`` argument;
conflicting declarations raise); other parameters follow the default rule.
A matrix block takes ``fraction`` of its rows per step when its smaller side is
at least ``selection_min_dim``, every row otherwise. Decayed groups carry no
``weight_decay`` key (they take the optimizer's); exempt groups carry 0.0.
AdamW groups come first, then matrix groups, each in parameter order.
"""

from __future__ import annotations

import logging
from collections.abc import Collection, Iterable, Mapping
from typing import Any, NamedTuple

from torch import Tensor, nn

from dionw_amd._buckets import block_shape
from dionw_amd._default_rule import Owner, default_route, is_exempt_from_decay, owners
from dionw_amd._keys import FRACTION_KEY, NUM_HEADS_KEY, ROUTE_KEY
from dionw_amd.report import RoutedParameter, RouteReason, RoutingReport
from dionw_amd.routing import Route, RouteKind, RouteProvider

__all__ = ["ROUTE_KEY", "ParamGroups", "param_groups"]

_LOGGER = logging.getLogger("dionw")


class ParamGroups(NamedTuple):
    """The groups for ``Dion`` and the report of how they were routed."""

    groups: list[dict[str, Any]]
    report: RoutingReport


def param_groups(
    model: nn.Module,
    *,
    params: Iterable[Tensor] | None = None,
    fraction: float = 0.25,
    selection_min_dim: int = 1024,
    min_matrix_dim: int = 8,
    routes: Mapping[Tensor, Route] | None = None,
    no_weight_decay: Collection[Tensor] | None = None,
) -> ParamGroups:
    """Route each trainable parameter of ``model`` and build ``Dion`` groups.

    Raises:
        ValueError: On out-of-range settings, invalid or conflicting routes,
            parameters not registered on ``model``, or nothing trainable.
    """
    if not 0.0 < fraction <= 1.0:
        raise ValueError(f"fraction must be in (0, 1], got {fraction}")
    if selection_min_dim <= 0 or min_matrix_dim <= 0:
        raise ValueError("selection_min_dim and min_matrix_dim must be positive")
    found = owners(model)
    trainable: dict[int, Tensor] = {}
    for param in model.parameters() if params is None else params:
        if param.requires_grad and id(param) not in trainable:
            trainable[id(param)] = param
    if not trainable:
        raise ValueError("No parameters require gradients")
    foreign = [tuple(p.shape) for key, p in trainable.items() if key not in found]
    if foreign:
        raise ValueError(f"Parameters not registered on the model: {foreign[:8]}")
    if no_weight_decay is None:
        exempt = {key for key, p in trainable.items() if is_exempt_from_decay(found[key], p)}
    else:
        exempt = {id(p) for p in no_weight_decay}
    declared = _declarations(model, routes)
    routed = [
        _resolve(
            found[key],
            param,
            declared.get(key),
            fraction,
            selection_min_dim,
            min_matrix_dim,
            decayed=key not in exempt,
        )
        for key, param in trainable.items()
    ]
    groups, report = _groups(list(trainable.values()), routed)
    _LOGGER.info("\n".join(report.lines()))
    return ParamGroups(groups=groups, report=report)


def _declarations(model: nn.Module, routes: Mapping[Tensor, Route] | None) -> dict[int, Route]:
    sources: list[tuple[str, Tensor, Route]] = [
        ("the routes argument", p, r) for p, r in (routes or {}).items()
    ]
    for module in model.modules():
        if isinstance(module, RouteProvider):
            sources.extend((type(module).__name__, p, r) for p, r in module.dion_routes())
    registered = {id(p) for p in model.parameters()}
    declared: dict[int, Route] = {}
    for source, param, route in sources:
        if id(param) not in registered:
            raise ValueError(
                f"{source} declares a route for a parameter (shape {tuple(param.shape)}) "
                "that is not registered on the model"
            )
        earlier = declared.setdefault(id(param), route)
        if earlier != route:
            raise ValueError(
                f"Conflicting routes for a parameter of shape {tuple(param.shape)}: "
                f"{earlier} vs {route} ({source})"
            )
    return declared


def _resolve(
    owner: Owner,
    param: Tensor,
    declared: Route | None,
    fraction: float,
    selection_min_dim: int,
    min_matrix_dim: int,
    *,
    decayed: bool,
) -> RoutedParameter:
    if declared is None:
        route, reason = default_route(owner, param, min_matrix_dim)
    else:
        route, reason = declared, RouteReason.DECLARED
    if route.kind is RouteKind.MATRIX:
        if param.ndim < 2:
            raise ValueError(
                f"MATRIX route on {owner.name} needs >= 2 dims, got {tuple(param.shape)}"
            )
        _, rows, cols = block_shape(param, route.num_heads)
        if route.fraction is not None:
            row_fraction = float(route.fraction)
        else:
            row_fraction = fraction if min(rows, cols) >= selection_min_dim else 1.0
    elif route.kind is RouteKind.ADAMW:
        row_fraction = 1.0
    else:
        raise RuntimeError(f"Unhandled RouteKind: {route.kind}")
    return RoutedParameter(
        name=owner.name,
        shape=tuple(int(d) for d in param.shape),
        kind=route.kind,
        fraction=row_fraction,
        num_heads=route.num_heads,
        decayed=decayed,
        reason=reason,
    )


def _groups(
    params: list[Tensor], routed: list[RoutedParameter]
) -> tuple[list[dict[str, Any]], RoutingReport]:
    buckets: dict[tuple[RouteKind, int | None, float, bool], list[int]] = {}
    for position, entry in enumerate(routed):
        key = (entry.kind, entry.num_heads, entry.fraction, entry.decayed)
        buckets.setdefault(key, []).append(position)
    # AdamW groups first; within a kind, first-seen order (a stable sort).
    ordered = sorted(buckets.items(), key=lambda item: item[0][0] is RouteKind.MATRIX)
    groups: list[dict[str, Any]] = []
    entries: list[RoutedParameter] = []
    for (kind, num_heads, row_fraction, decayed), positions in ordered:
        group: dict[str, Any] = {"params": [params[i] for i in positions], ROUTE_KEY: kind.value}
        if kind is RouteKind.MATRIX:
            group[FRACTION_KEY] = row_fraction
            group[NUM_HEADS_KEY] = num_heads
        if not decayed:
            group["weight_decay"] = 0.0
        groups.append(group)
        entries.extend(routed[i] for i in positions)
    return groups, RoutingReport(tuple(entries))
