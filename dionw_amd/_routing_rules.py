"""Default routing of the parameters nothing declared, as a rule table.

The rules are tried in order and the first that claims a parameter sends it to
AdamW with its reason; a parameter no rule claims is a MATRIX. The order and
what each rule matches are the reference's routing contract
(_default_rule.py:67-127): an ``nn.Embedding``/``EmbeddingBag`` weight, a
grouped convolution's weight, a learned token set (own name ending in
``token``/``tokens``), an embedding-like own name, a vector or scalar, a
tensor whose smaller side (trailing dims flattened into columns) is below
``min_matrix_dim``. Vectors, learned token sets and embedding-like names are
also exempt from weight decay; ``nn.Embedding`` weights are decayed.
"""

from __future__ import annotations

import math
from collections.abc import Callable
from dataclasses import dataclass
from typing import Final

from torch import Tensor, nn

from dionw_amd.report import RouteReason
from dionw_amd.routing import Route, RouteKind

__all__ = ["Site", "decay_exempt", "default_route", "sites"]

TOKEN_SUFFIXES: Final = ("token", "tokens")
EMBEDDING_NAME_PARTS: Final = ("pos_embed", "position_embedding", "relative_position_bias")
_CONVOLUTIONS: Final = (nn.Conv1d, nn.Conv2d, nn.Conv3d,
                        nn.ConvTranspose1d, nn.ConvTranspose2d, nn.ConvTranspose3d)


@dataclass(frozen=True)
class Site:
    """Where a parameter is first registered.

    Attributes:
        path: Qualified name (``layers.0.attn.weight``).
        module: The module that holds it.
        attr: Its own name in that module.
    """

    path: str
    module: nn.Module
    attr: str


def sites(model: nn.Module) -> dict[int, Site]:
    """The first registration of every parameter of ``model``, by ``id``."""
    found: dict[int, Site] = {}
    for prefix, module in model.named_modules():
        for attr, param in module.named_parameters(recurse=False):
            found.setdefault(id(param), Site(f"{prefix}.{attr}" if prefix else attr, module, attr))
    return found


def _smaller_side(param: Tensor) -> int:
    return min(int(param.shape[0]), math.prod(int(d) for d in param.shape[1:]))


def _tokens(site: Site) -> bool:
    return site.attr.endswith(TOKEN_SUFFIXES)


def _embedding_named(site: Site) -> bool:
    return any(part in site.attr for part in EMBEDDING_NAME_PARTS)


# (reason, predicate of (site, parameter, min_matrix_dim)), first match wins.
_ADAMW_RULES: Final[tuple[tuple[RouteReason, Callable[[Site, Tensor, int], bool]], ...]] = (
    (RouteReason.EMBEDDING,
     lambda s, p, d: s.attr == "weight" and isinstance(s.module, (nn.Embedding, nn.EmbeddingBag))),
    (RouteReason.GROUPED_CONVOLUTION,
     lambda s, p, d: s.attr == "weight" and isinstance(s.module, _CONVOLUTIONS)
     and int(s.module.groups) > 1),
    (RouteReason.LEARNED_TOKENS, lambda s, p, d: _tokens(s)),
    (RouteReason.EMBEDDING_NAME, lambda s, p, d: _embedding_named(s)),
    (RouteReason.VECTOR, lambda s, p, d: p.ndim < 2),
    (RouteReason.NARROW, lambda s, p, d: _smaller_side(p) < d),
)


def default_route(site: Site, param: Tensor, min_matrix_dim: int) -> tuple[Route, RouteReason]:
    """The route of an undeclared parameter and the rule that chose it."""
    for reason, claims in _ADAMW_RULES:
        if claims(site, param, min_matrix_dim):
            return Route(RouteKind.ADAMW), reason
    return Route(RouteKind.MATRIX), RouteReason.MATRIX


def decay_exempt(site: Site, param: Tensor) -> bool:
    """Whether the default decay rule exempts the parameter."""
    return param.ndim < 2 or _tokens(site) or _embedding_named(site)
