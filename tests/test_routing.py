"""Parameter routing on the CPU: the default rule, declared routes, row
fractions, weight-decay groups and the report.

The expected outcomes are those the reference's routing tests fix
(tests/test_routing.py:19-214; rules in _default_rule.py:67-127 and
param_groups.py:89-270), checked here on models of this file's own making.
"""

from __future__ import annotations

import pytest
import torch
from torch import nn

from dionw_amd import ROUTE_KEY, Route, RouteKind, param_groups
from dionw_amd.report import RouteReason as Why

M, A = RouteKind.MATRIX, RouteKind.ADAMW
SIZES = {"fraction": 0.5, "selection_min_dim": 1024, "min_matrix_dim": 8}


def _zoo() -> nn.Module:
    """A module holding one parameter per outcome of the default rule."""
    zoo = nn.Module()
    zoo.plain = nn.Parameter(torch.zeros(24, 40))                   # a bare 2-D parameter
    zoo.attn = nn.MultiheadAttention(16, 2, batch_first=True)       # in_proj_* and out_proj
    zoo.deconv = nn.ConvTranspose2d(16, 8, 2, stride=2)
    zoo.conv = nn.Conv2d(16, 8, 3)
    zoo.depthwise = nn.Conv2d(16, 16, 3, groups=16)
    zoo.tok = nn.Embedding(50, 16)
    zoo.pos_embed = nn.Parameter(torch.zeros(10, 16))               # an embedding by name
    zoo.register_tokens = nn.Parameter(torch.zeros(4, 16))          # learned tokens by name
    zoo.head = nn.Linear(16, 3)                                     # 3 < min_matrix_dim
    zoo.ln = nn.LayerNorm(16)
    zoo.pos_embedder = nn.Linear(16, 16, bias=False)                # its own name is "weight"
    return zoo


OUTCOMES = {
    "plain": (M, Why.MATRIX),
    "attn.in_proj_weight": (M, Why.MATRIX),
    "attn.in_proj_bias": (A, Why.VECTOR),
    "attn.out_proj.weight": (M, Why.MATRIX),
    "attn.out_proj.bias": (A, Why.VECTOR),
    "deconv.weight": (M, Why.MATRIX),
    "deconv.bias": (A, Why.VECTOR),
    "conv.weight": (M, Why.MATRIX),
    "conv.bias": (A, Why.VECTOR),
    "depthwise.weight": (A, Why.GROUPED_CONVOLUTION),
    "depthwise.bias": (A, Why.VECTOR),
    "tok.weight": (A, Why.EMBEDDING),
    "pos_embed": (A, Why.EMBEDDING_NAME),
    "register_tokens": (A, Why.LEARNED_TOKENS),
    "head.weight": (A, Why.NARROW),
    "head.bias": (A, Why.VECTOR),
    "ln.weight": (A, Why.VECTOR),
    "ln.bias": (A, Why.VECTOR),
    "pos_embedder.weight": (M, Why.MATRIX),
}


def test_every_default_rule_outcome() -> None:
    """Each parameter of the zoo takes the route and reason of the table."""
    _, report = param_groups(_zoo(), **SIZES)
    assert {e.name: (e.kind, e.reason) for e in report.parameters} == OUTCOMES


class _HeadsAndPatches(nn.Module):
    """Declares its routes through ``dion_routes`` alone (no base class)."""

    def __init__(self) -> None:
        super().__init__()
        self.fused_qkv = nn.Linear(32, 96, bias=False)
        self.stem = nn.Linear(24, 32, bias=False)

    def dion_routes(self):
        yield self.fused_qkv.weight, Route(M, num_heads=6)
        yield self.stem.weight, Route(A)


def test_declared_routes_split_heads_and_force_adamw() -> None:
    model = _HeadsAndPatches()
    groups, report = param_groups(model, **SIZES)
    entries = {e.name: e for e in report.parameters}
    qkv = entries["fused_qkv.weight"]
    assert (qkv.kind, qkv.reason, qkv.num_heads) == (M, Why.DECLARED, 6)
    assert entries["stem.weight"].kind is A
    (matrix_group,) = [g for g in groups if g[ROUTE_KEY] == M.value]
    assert matrix_group["num_heads"] == 6 and matrix_group["params"] == [model.fused_qkv.weight]


@pytest.mark.parametrize(("route", "stranger", "fragment"), [
    (Route(A), False, "Conflicting routes"),
    (Route(A), True, "not registered"),
])
def test_routes_argument_conflicts(route, stranger, fragment) -> None:
    """An argument route that contradicts a module's declaration, or names a
    parameter the model does not own, is refused; an agreeing one merges."""
    model = _HeadsAndPatches()
    agreeing = {model.fused_qkv.weight: Route(M, num_heads=6)}
    assert param_groups(model, routes=agreeing, **SIZES).report.parameters
    target = nn.Parameter(torch.zeros(4, 4)) if stranger else model.fused_qkv.weight
    with pytest.raises(ValueError, match=fragment):
        param_groups(model, routes={target: route}, **SIZES)


def test_selection_starts_at_selection_min_dim_and_a_declared_fraction_wins() -> None:
    model = nn.Module()
    model.big = nn.Linear(40, 72, bias=False)      # smaller side 40 >= 32: rows selected
    model.small = nn.Linear(12, 72, bias=False)    # smaller side 12 < 32: every row
    model.pinned = nn.Linear(40, 40, bias=False)   # declared fraction 1
    _, report = param_groups(model, fraction=0.25, selection_min_dim=32, min_matrix_dim=8,
                             routes={model.pinned.weight: Route(M, fraction=1.0)})
    got = {e.name: e.fraction for e in report.parameters}
    assert got == {"big.weight": 0.25, "small.weight": 1.0, "pinned.weight": 1.0}


def test_decay_groups_inherit_the_optimizer_value() -> None:
    """Decayed groups carry no weight_decay (the optimizer's applies), exempt ones
    0.0; ``no_weight_decay`` replaces the default choice of exempt parameters."""
    zoo = _zoo()
    groups, report = param_groups(zoo, **SIZES)
    decayed = {e.name for e in report.parameters if e.decayed}
    assert {"plain", "tok.weight", "conv.weight"} <= decayed
    assert not decayed & {"ln.weight", "conv.bias", "pos_embed", "register_tokens"}
    name_of = {id(p): n for n, p in zoo.named_parameters()}
    for group in groups:
        flags = {name_of[id(p)] in decayed for p in group["params"]}
        assert flags in ({True}, {False})
        assert group.get("weight_decay") == (None if flags == {True} else 0.0)
    _, only_plain = param_groups(zoo, no_weight_decay=[zoo.plain], **SIZES)
    assert [e.name for e in only_plain.parameters if not e.decayed] == ["plain"]


def test_adamw_groups_come_first_and_frozen_parameters_are_left_out() -> None:
    zoo = _zoo()
    zoo.conv.requires_grad_(False)
    groups, report = param_groups(zoo, **SIZES)
    kinds = [RouteKind(g[ROUTE_KEY]) for g in groups]
    assert kinds == sorted(kinds, key=lambda k: k is M)
    assert all(not e.name.startswith("conv.") for e in report.parameters)
    text = report.lines()
    assert text[0] == "dionw parameter routing:"
    assert "    adamw (learned tokens): register_tokens (4, 16)" in text


def test_out_of_range_settings_are_refused() -> None:
    zoo = _zoo()
    with pytest.raises(ValueError, match="fraction"):
        param_groups(zoo, **{**SIZES, "fraction": 0.0})
    zoo.requires_grad_(False)
    with pytest.raises(ValueError, match="No parameters require gradients"):
        param_groups(zoo, **SIZES)
    with pytest.raises(ValueError, match="MATRIX routes"):
        Route(A, num_heads=2)
