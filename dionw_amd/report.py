"""The routing report (reference: src/dionw/report.py:14-82)."""

from __future__ import annotations

import math
from dataclasses import dataclass
from enum import Enum

from dionw_amd.routing import RouteKind

__all__ = ["RouteReason", "RoutedParameter", "RoutingReport"]


class RouteReason(Enum):
    """The rule of the default routing (or a declaration) that chose a route."""

    DECLARED = "declared"
    EMBEDDING = "embedding"
    GROUPED_CONVOLUTION = "grouped convolution"
    LEARNED_TOKENS = "learned tokens"
    EMBEDDING_NAME = "embedding-like name"
    VECTOR = "vector"
    NARROW = "narrow"
    MATRIX = "matrix"


@dataclass(frozen=True)
class RoutedParameter:
    """One parameter's resolved route, row fraction, head split and decay."""

    name: str
    shape: tuple[int, ...]
    kind: RouteKind
    fraction: float
    num_heads: int | None
    decayed: bool
    reason: RouteReason


@dataclass(frozen=True)
class RoutingReport:
    """One entry per routed parameter, ordered as the groups list them."""

    parameters: tuple[RoutedParameter, ...]

    def lines(self) -> list[str]:
        """A summary: one line per group, then each >=2-D AdamW parameter and why."""
        totals: dict[tuple[RouteKind, float, int | None, bool], list[int]] = {}
        for p in self.parameters:
            totals.setdefault((p.kind, p.fraction, p.num_heads, p.decayed), []).append(
                math.prod(p.shape)
            )
        out = ["dionw parameter routing:"]
        for (kind, fraction, heads, decayed), sizes in totals.items():
            out.append(
                f"  {kind.value} fraction={fraction} heads={heads} "
                f"decay={'yes' if decayed else 'no'} tensors={len(sizes)} "
                f"params={sum(sizes) / 1e6:.2f}M"
            )
        for p in self.parameters:
            if p.kind is RouteKind.ADAMW and len(p.shape) >= 2:
                out.append(f"    adamw ({p.reason.value}): {p.name} {p.shape}")
        return out
