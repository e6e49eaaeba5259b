"""``param_groups(model)``: route every trainable parameter and build Dion groups.

A ``_Router`` indexes the model once (where each parameter is registered, the
routes its ``RouteProvider`` modules and the ``routes`` argument declare) and
decides each parameter: a declared route wins over the default rule table
(``_routing_rules``); a MATRIX parameter takes ``fraction`` of its blocks'
rows per step when the blocks' smaller side is at least ``selection_min_dim``,
every row otherwise, unless its route fixes the fraction. The decisions are
then laid out as groups — AdamW groups first, then matrix groups, each group
one combination of (route, heads, fraction, decay) in order of first
appearance, parameters in their given order. Decayed groups carry no
``weight_decay`` (they take the optimizer's), exempt ones carry 0.0. The
outcome and the error messages are the reference's (param_groups.py:89-270).
"""

from __future__ import annotations

import logging
from collections.abc import Collection, Iterable, Mapping
from typing import Any, NamedTuple

from torch import Tensor, nn

from dionw_amd._groups import matrix_blocks
from dionw_amd._keys import FRACTION_KEY, NUM_HEADS_KEY, ROUTE_KEY
from dionw_amd._routing_rules import Site, decay_exempt, default_route, sites
from dionw_amd.report import RoutedParameter, RouteReason, RoutingReport
from dionw_amd.routing import Route, RouteKind, RouteProvider

__all__ = ["ROUTE_KEY", "ParamGroups", "param_groups"]

_LOG = logging.getLogger("dionw")


class ParamGroups(NamedTuple):
    """The groups for ``Dion`` and the report of how they were routed."""

    groups: list[dict[str, Any]]
    report: RoutingReport


class _Router:
    """Routes the parameters of one model under one set of settings."""

    def __init__(self, model: nn.Module, *, fraction: float, selection_min_dim: int,
                 min_matrix_dim: int, routes: Mapping[Tensor, Route] | None) -> None:
        if not 0.0 < fraction <= 1.0:
            raise ValueError(f"the row fraction {fraction} lies outside (0, 1]")
        if selection_min_dim <= 0 or min_matrix_dim <= 0:
            raise ValueError("selection_min_dim and min_matrix_dim must be at least 1")
        self.fraction = fraction
        self.selection_min_dim = selection_min_dim
        self.min_matrix_dim = min_matrix_dim
        self.sites = sites(model)
        self.declared = self._collect_declarations(model, routes)

    def _collect_declarations(self, model: nn.Module,
                              routes: Mapping[Tensor, Route] | None) -> dict[int, Route]:
        """Declared routes by parameter id; a declaration must name a parameter
        of the model, and two declarations of one parameter must agree."""
        claims: list[tuple[str, Tensor, Route]] = [
            ("the routes argument", param, route) for param, route in (routes or {}).items()]
        for module in model.modules():
            if isinstance(module, RouteProvider):
                claims += [(type(module).__name__, p, r) for p, r in module.dion_routes()]
        declared: dict[int, Route] = {}
        for source, param, route in claims:
            if id(param) not in self.sites:
                raise ValueError(f"{source} routes a parameter of shape {tuple(param.shape)} "
                                 "that the model has not registered")
            known = declared.get(id(param))
            if known is not None and known != route:
                raise ValueError(f"Conflicting routes: {known} and {route} ({source}) both "
                                 f"claim the parameter of shape {tuple(param.shape)}")
            declared[id(param)] = route
        return declared

    def decide(self, param: Tensor, decayed: bool) -> RoutedParameter:
        """One parameter's route, row fraction, head split and decay."""
        site: Site = self.sites[id(param)]
        route = self.declared.get(id(param))
        if route is None:
            route, reason = default_route(site, param, self.min_matrix_dim)
        else:
            reason = RouteReason.DECLARED
        if route.kind is RouteKind.ADAMW:
            rows_fraction = 1.0
        elif route.kind is RouteKind.MATRIX:
            if param.ndim < 2:
                raise ValueError(f"MATRIX route on {site.path} needs >= 2 dims, got "
                                 f"{tuple(param.shape)}")
            _, rows, cols = matrix_blocks(param, route.num_heads)
            if route.fraction is not None:
                rows_fraction = float(route.fraction)
            elif min(rows, cols) >= self.selection_min_dim:
                rows_fraction = self.fraction
            else:
                rows_fraction = 1.0
        else:
            raise RuntimeError(f"Unhandled RouteKind: {route.kind}")
        return RoutedParameter(name=site.path, shape=tuple(int(d) for d in param.shape),
                               kind=route.kind, fraction=rows_fraction,
                               num_heads=route.num_heads, decayed=decayed, reason=reason)


def _layout(params: list[Tensor], decisions: list[RoutedParameter]) -> ParamGroups:
    """Groups (AdamW first, then MATRIX; each by first appearance) and the
    report in the same order."""
    slots: dict[tuple[Any, ...], list[int]] = {}
    for i, d in enumerate(decisions):
        slots.setdefault((d.kind is RouteKind.MATRIX, d.kind, d.num_heads, d.fraction,
                          d.decayed), []).append(i)
    groups: list[dict[str, Any]] = []
    order: list[int] = []
    for key in sorted(slots, key=lambda k: k[0]):  # stable: first appearance within a kind
        members = slots[key]
        _, kind, num_heads, fraction, decayed = key
        group: dict[str, Any] = {"params": [params[i] for i in members], ROUTE_KEY: kind.value}
        if kind is RouteKind.MATRIX:
            group.update({FRACTION_KEY: fraction, NUM_HEADS_KEY: num_heads})
        if not decayed:
            group["weight_decay"] = 0.0
        groups.append(group)
        order += members
    return ParamGroups(groups, RoutingReport(tuple(decisions[i] for i in order)))


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

    Args:
        model: Owns the parameters; its ``RouteProvider`` modules declare routes.
        params: The parameters to optimize (None: all of ``model``'s); those
            without ``requires_grad`` are skipped.
        fraction: Row fraction of blocks whose smaller side is at least
            ``selection_min_dim``, in (0, 1].
        selection_min_dim: Smaller side from which blocks select rows.
        min_matrix_dim: Smaller side below which tensors take AdamW.
        routes: Extra per-parameter routes, merged with the modules' own.
        no_weight_decay: Exactly the parameters exempt from weight decay (None:
            the default rule).

    Returns:
        ``(groups, report)``; the report is also logged at INFO on ``dionw``.

    Raises:
        ValueError: For out-of-range settings, invalid or conflicting routes,
            parameters not registered on ``model``, or nothing trainable.
    """
    router = _Router(model, fraction=fraction, selection_min_dim=selection_min_dim,
                     min_matrix_dim=min_matrix_dim, routes=routes)
    chosen = list({id(p): p for p in (model.parameters() if params is None else params)
                   if p.requires_grad}.values())
    if not chosen:
        raise ValueError("No parameters require gradients")
    outside = [tuple(p.shape) for p in chosen if id(p) not in router.sites]
    if outside:
        raise ValueError(f"{len(outside)} of the given parameters are not registered on the model, for instance shapes {outside[:8]}")
    exempt = ({id(p) for p in chosen if decay_exempt(router.sites[id(p)], p)}
              if no_weight_decay is None else {id(p) for p in no_weight_decay})
    decisions = [router.decide(p, id(p) not in exempt) for p in chosen]
    result = _layout(chosen, decisions)
    _LOG.info("\n".join(result.report.lines()))
    return result
