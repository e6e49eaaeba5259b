"""Options of the Dion update of a matrix: which iteration, which row scaling, which momentum.

Reference: src/dionw/matrix_update.py:26-73. ``DION3_UPDATE`` (the default) is
row-selected NorMuon with heavy-ball momentum; ``MUON_UPDATE`` is Keller
Jordan's Muon (Nesterov momentum, no row normalization) for groups that update
every row.
"""

from __future__ import annotations

from dataclasses import dataclass
from enum import Enum
from typing import Final

from dionw_amd.newton_schulz import NewtonSchulz

__all__ = ["DION3_UPDATE", "MUON_UPDATE", "MatrixUpdate", "MomentumForm", "RowNormalization"]


class RowNormalization(Enum):
    """Post-processing of the orthogonalized rows before they are applied."""

    NORMUON = "normuon"  # divide rows by the root of an EMA of their mean square
    NONE = "none"        # use the orthogonalized update as is


class MomentumForm(Enum):
    """Which momentum is orthogonalized: ``B`` (heavy ball) or ``G + mu B`` (Nesterov)."""

    HEAVY_BALL = "heavy_ball"
    NESTEROV = "nesterov"


@dataclass(frozen=True)
class MatrixUpdate:
    """The three choices that define a matrix update: iteration, row scaling, momentum."""

    newton_schulz: NewtonSchulz
    row_normalization: RowNormalization
    momentum_form: MomentumForm


DION3_UPDATE: Final = MatrixUpdate(
    NewtonSchulz.GRAM, RowNormalization.NORMUON, MomentumForm.HEAVY_BALL
)
MUON_UPDATE: Final = MatrixUpdate(
    NewtonSchulz.KELLER_TRITON, RowNormalization.NONE, MomentumForm.NESTEROV
)
