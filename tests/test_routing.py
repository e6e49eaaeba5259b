"""Parameter routing (CPU): the default rule, declared routes, row fractions,
weight-decay groups and the report, against the outcomes the reference's own
routing tests fix (tests/test_routing.py:19-214; _default_rule.py:67-127;
param_groups.py:89-270). Routing is host logic: the models stay on the CPU."""

from __future__ import annotations

from collections.abc import Iterable

import pytest
import torch
from torch import Tensor, nn

from dionw_amd import ROUTE_KEY, Route, RouteKind, param_groups
from dionw_amd.report import RouteReason

MATRIX, ADAMW = RouteKind.MATRIX, RouteKind.ADAMW


class _EveryOutcome(nn.Module):
    """One parameter for each outcome of the default rule."""

    def __init__(self) -> None:
        super().__init__()
        self.bare = nn.Parameter(torch.zeros(32, 48))
        self.mha = nn.MultiheadAttention(32, 4, batch_first=True)
        self.up = nn.ConvTranspose2d(32, 16, 2, stride=2)
        self.conv = nn.Conv2d(32, 16, 3)
        self.grouped = nn.Conv2d(32, 32, 3, groups=4)
        self.embed = nn.Embedding(64, 32)
        self.pos_embed = nn.Parameter(torch.zeros(16, 32))
        self.register_tokens = nn.Parameter(torch.zeros(16, 32))
        self.narrow = nn.Linear(32, 4)
        self.norm = nn.LayerNorm(32)
        # The name rules read a parameter's own name ("weight"), not its module's.
        self.pos_embedder = nn.Linear(32, 32, bias=False)


def _routes(model: nn.Module, **kwargs) -> dict[str, tuple[RouteKind, RouteReason]]:
    _, report = param_groups(model, **kwargs)
    return {p.name: (p.kind, p.reason) for p in report.parameters}


def test_default_rule_outcomes() -> None:
    """tests/test_routing.py:38-63."""
    got = _routes(_EveryOutcome(), fraction=0.5, selection_min_dim=1024, min_matrix_dim=8)
    assert got == {
        "bare": (MATRIX, RouteReason.MATRIX),
        "mha.in_proj_weight": (MATRIX, RouteReason.MATRIX),
        "mha.in_proj_bias": (ADAMW, RouteReason.VECTOR),
        "mha.out_proj.weight": (MATRIX, RouteReason.MATRIX),
        "mha.out_proj.bias": (ADAMW, RouteReason.VECTOR),
        "up.weight": (MATRIX, RouteReason.MATRIX),
        "up.bias": (ADAMW, RouteReason.VECTOR),
        "conv.weight": (MATRIX, RouteReason.MATRIX),
        "conv.bias": (ADAMW, RouteReason.VECTOR),
        "grouped.weight": (ADAMW, RouteReason.GROUPED_CONVOLUTION),
        "grouped.bias": (ADAMW, RouteReason.VECTOR),
        "embed.weight": (ADAMW, RouteReason.EMBEDDING),
        "pos_embed": (ADAMW, RouteReason.EMBEDDING_NAME),
        "register_tokens": (ADAMW, RouteReason.LEARNED_TOKENS),
        "narrow.weight": (ADAMW, RouteReason.NARROW),
        "narrow.bias": (ADAMW, RouteReason.VECTOR),
        "norm.weight": (ADAMW, RouteReason.VECTOR),
        "norm.bias": (ADAMW, RouteReason.VECTOR),
        "pos_embedder.weight": (MATRIX, RouteReason.MATRIX),
    }


class _Declares(nn.Module):
    """Declares routes without inheriting anything (the provider is a protocol)."""

    def __init__(self) -> None:
        super().__init__()
        self.qkv = nn.Linear(64, 192, bias=False)
        self.patch = nn.Linear(48, 64, bias=False)

    def dion_routes(self) -> Iterable[tuple[Tensor, Route]]:
        return ((self.qkv.weight, Route(MATRIX, num_heads=6)), (self.patch.weight, Route(ADAMW)))


def test_declarations_route_and_split_heads() -> None:
    """tests/test_routing.py:80-92."""
    model = _Declares()
    groups, report = param_groups(model, fraction=0.5, selection_min_dim=1024, min_matrix_dim=8)
    by_name = {p.name: p for p in report.parameters}
    assert by_name["qkv.weight"].num_heads == 6
    assert by_name["qkv.weight"].reason is RouteReason.DECLARED
    assert by_name["patch.weight"].kind is ADAMW
    matrix = next(g for g in groups if g[ROUTE_KEY] == MATRIX.value)
    assert matrix["num_heads"] == 6 and matrix["params"] == [model.qkv.weight]


def test_routes_argument_merges_and_conflicts_raise() -> None:
    """tests/test_routing.py:95-117: an agreeing route merges, a clash or a
    parameter the model does not own raises."""
    model = _Declares()
    kwargs = {"fraction": 0.5, "selection_min_dim": 1024, "min_matrix_dim": 8}
    same = {model.qkv.weight: Route(MATRIX, num_heads=6)}
    assert param_groups(model, routes=same, **kwargs).report.parameters
    with pytest.raises(ValueError, match="Conflicting routes"):
        param_groups(model, routes={model.qkv.weight: Route(ADAMW)}, **kwargs)
    stranger = nn.Parameter(torch.zeros(8, 8))
    with pytest.raises(ValueError, match="not registered"):
        param_groups(model, routes={stranger: Route(ADAMW)}, **kwargs)


class _Fractions(nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.wide = nn.Linear(64, 96, bias=False)
        self.narrow = nn.Linear(16, 96, bias=False)
        self.declared = nn.Linear(64, 64, bias=False)


def test_row_fraction_applies_from_selection_min_dim() -> None:
    """tests/test_routing.py:127-141: rows are selected from selection_min_dim
    on (smaller side 64 >= 32 selects, 16 does not); a declared fraction wins."""
    model = _Fractions()
    routes = {model.declared.weight: Route(MATRIX, fraction=1.0)}
    _, report = param_groups(model, fraction=0.25, selection_min_dim=32, min_matrix_dim=8,
                             routes=routes)
    assert {p.name: p.fraction for p in report.parameters} == {
        "wide.weight": 0.25, "narrow.weight": 1.0, "declared.weight": 1.0}


def test_weight_decay_groups_inherit_the_optimizer_value() -> None:
    """tests/test_routing.py:144-174: decayed groups carry no weight_decay key
    (they inherit the optimizer's), exempt groups carry 0.0, and
    no_weight_decay replaces the default rule."""
    model = _EveryOutcome()
    kwargs = {"fraction": 0.5, "selection_min_dim": 1024, "min_matrix_dim": 8}
    groups, report = param_groups(model, **kwargs)
    decayed = {p.name for p in report.parameters if p.decayed}
    assert {"bare", "embed.weight", "conv.weight"} <= decayed
    assert {"norm.weight", "conv.bias", "pos_embed", "register_tokens"}.isdisjoint(decayed)
    names = {id(p): n for n, p in model.named_parameters()}
    for group in groups:
        flags = {names[id(p)] in decayed for p in group["params"]}
        assert len(flags) == 1
        if flags == {True}:
            assert "weight_decay" not in group
        else:
            assert group["weight_decay"] == 0.0
    _, explicit = param_groups(model, no_weight_decay=[model.bare], **kwargs)
    assert {p.name for p in explicit.parameters if not p.decayed} == {"bare"}


def test_groups_order_adamw_first_and_skip_frozen_parameters() -> None:
    """tests/test_routing.py:177-190."""
    model = _EveryOutcome()
    model.conv.requires_grad_(False)
    groups, report = param_groups(model, fraction=0.5, selection_min_dim=1024, min_matrix_dim=8)
    kinds = [RouteKind(g[ROUTE_KEY]) for g in groups]
    first_matrix = kinds.index(MATRIX)
    assert set(kinds[:first_matrix]) == {ADAMW} and set(kinds[first_matrix:]) == {MATRIX}
    assert not any(p.name.startswith("conv.") for p in report.parameters)
    lines = report.lines()
    assert lines[0] == "dionw parameter routing:"
    assert "    adamw (learned tokens): register_tokens (16, 32)" in lines


def test_invalid_settings_raise() -> None:
    """tests/test_routing.py:193-202."""
    model = _EveryOutcome()
    with pytest.raises(ValueError, match="fraction"):
        param_groups(model, fraction=0.0, selection_min_dim=1024, min_matrix_dim=8)
    model.requires_grad_(False)
    with pytest.raises(ValueError, match="No parameters require gradients"):
        param_groups(model, fraction=0.5, selection_min_dim=1024, min_matrix_dim=8)
    with pytest.raises(ValueError, match="MATRIX routes"):
        Route(ADAMW, num_heads=2)
