"""Default route and weight-decay rules (reference: src/dionw/_default_rule.py:52-127).

First match wins: embedding weights, grouped-convolution weights, learned
token sets (own name ending in ``token``/``tokens``), embedding-like names,
vectors/scalars, narrow tensors (smaller side below ``min_matrix_dim``) take
AdamW; everything else is a MATRIX.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Final

from torch import Tensor, nn

from dionw_amd.report import RouteReason
from dionw_amd.routing import Route, RouteKind

__all__ = [
    "EMBEDDING_NAME_SUBSTRINGS",
    "LEARNED_TOKEN_NAME_SUFFIXES",
    "Owner",
    "default_route",
    "is_exempt_from_decay",
    "matrix_dims",
    "owners",
]

LEARNED_TOKEN_NAME_SUFFIXES: Final = ("token", "tokens")
EMBEDDING_NAME_SUBSTRINGS: Final = ("pos_embed", "position_embedding", "relative_position_bias")
_CONVS: Final = (
    nn.Conv1d,
    nn.Conv2d,
    nn.Conv3d,
    nn.ConvTranspose1d,
    nn.ConvTranspose2d,
    nn.ConvTranspose3d,
)


@dataclass(frozen=True)
class Owner:
    """Where a parameter is registered: qualified name, module, local name."""

    name: str
    module: nn.Module
    local_name: str


def owners(model: nn.Module) -> dict[int, Owner]:
    """Each parameter's first registration, keyed by ``id(parameter)``."""
    found: dict[int, Owner] = {}
    for prefix, module in model.named_modules():
        for local, param in module.named_parameters(recurse=False):
            if id(param) not in found:
                found[id(param)] = Owner(f"{prefix}.{local}" if prefix else local, module, local)
    return found


def matrix_dims(param: Tensor) -> tuple[int, int]:
    """``(rows, cols)`` of a tensor read as a matrix (trailing dims flattened)."""
    return int(param.shape[0]), math.prod(int(d) for d in param.shape[1:])


def _embedding_name(local_name: str) -> bool:
    return any(part in local_name for part in EMBEDDING_NAME_SUBSTRINGS)


def _module_reason(owner: Owner) -> RouteReason | None:
    if owner.local_name != "weight":
        return None
    module = owner.module
    if isinstance(module, (nn.Embedding, nn.EmbeddingBag)):
        return RouteReason.EMBEDDING
    if isinstance(module, _CONVS) and int(module.groups) > 1:
        return RouteReason.GROUPED_CONVOLUTION
    return None


def default_route(owner: Owner, param: Tensor, min_matrix_dim: int) -> tuple[Route, RouteReason]:
    """The route of a parameter nothing declared, and the rule that chose it."""
    reason = _module_reason(owner)
    if reason is None:
        if owner.local_name.endswith(LEARNED_TOKEN_NAME_SUFFIXES):
            reason = RouteReason.LEARNED_TOKENS
        elif _embedding_name(owner.local_name):
            reason = RouteReason.EMBEDDING_NAME
        elif param.ndim < 2:
            reason = RouteReason.VECTOR
        elif min(matrix_dims(param)) < min_matrix_dim:
            reason = RouteReason.NARROW
    if reason is None:
        return Route(RouteKind.MATRIX), RouteReason.MATRIX
    return Route(RouteKind.ADAMW), reason


def is_exempt_from_decay(owner: Owner, param: Tensor) -> bool:
    """Vectors, learned token sets and embedding-like names skip weight decay."""
    return (
        param.ndim < 2
        or owner.local_name.endswith(LEARNED_TOKEN_NAME_SUFFIXES)
        or _embedding_name(owner.local_name)
    )
