"""Per-parameter routes (reference: src/dionw/routing.py:22-83).

``param_groups`` routes every parameter by a default rule; a module overrides
it for its own parameters with a ``dion_routes`` method (``RouteProvider``),
or the caller passes a ``routes`` mapping.
"""

from __future__ import annotations

from collections.abc import Iterable
from dataclasses import dataclass
from enum import Enum
from typing import Protocol, runtime_checkable

from torch import Tensor

__all__ = ["Route", "RouteKind", "RouteProvider"]


class RouteKind(Enum):
    """The two updates a parameter can get: Dion on a matrix, or AdamW."""

    ADAMW = "adamw"    # element-wise AdamW
    MATRIX = "matrix"  # the orthogonalized, row-selected matrix update


@dataclass(frozen=True)
class Route:
    """Where one parameter goes (Dion or AdamW) and, for Dion, with which options.

    Attributes:
        kind: The update.
        num_heads: MATRIX only: orthogonalize this many equal row blocks
            separately (None: the whole matrix).
        fraction: MATRIX only: share of each block's rows updated per step,
            overriding the size rule (None: the rule).

    Raises:
        ValueError: For matrix options on an AdamW route or out-of-range values.
    """

    kind: RouteKind
    num_heads: int | None = None
    fraction: float | None = None

    def __post_init__(self) -> None:
        if self.kind is RouteKind.ADAMW:
            if self.num_heads is not None or self.fraction is not None:
                raise ValueError("num_heads and fraction are options of MATRIX routes, not of AdamW ones")
        elif self.kind is RouteKind.MATRIX:
            if self.num_heads is not None and self.num_heads <= 0:
                raise ValueError(f"a route splits into at least one head, not {self.num_heads}")
            if self.fraction is not None and not 0.0 < self.fraction <= 1.0:
                raise ValueError(f"a route's row fraction {self.fraction} lies outside (0, 1]")
        else:
            raise RuntimeError(f"Unhandled RouteKind: {self.kind}")


@runtime_checkable
class RouteProvider(Protocol):
    """A module declaring routes for some of its own parameters."""

    def dion_routes(self) -> Iterable[tuple[Tensor, Route]]:
        """Each parameter this module routes itself, with its route."""
        ...
