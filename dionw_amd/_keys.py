"""Names of Dion's param-group and per-parameter state entries.

These strings are the checkpoint contract of the reference (src/dionw/_keys.py:
33-68): a state dict saved by either implementation loads in the other.
the group keys torch itself uses (``params``, ``lr``, ``betas``, ``eps``,
``weight_decay``) keep torch's spelling.
"""

from __future__ import annotations

from collections.abc import MutableMapping
from typing import Any, Final

from torch import Tensor

ParamState = MutableMapping[Tensor, dict[str, Any]]

# Param-group keys.
ROUTE_KEY: Final = "dion_route"                  # a RouteKind value
NEWTON_SCHULZ_KEY: Final = "newton_schulz"       # a NewtonSchulz value
FRACTION_KEY: Final = "fraction"                 # share of rows updated per step
NUM_HEADS_KEY: Final = "num_heads"               # row split of each matrix, or None
MOMENTUM_KEY: Final = "momentum"                 # matrix momentum (error-feedback decay)
MUON_BETA2_KEY: Final = "muon_beta2"             # NorMuon second-moment decay
ROW_NORMALIZATION_KEY: Final = "row_normalization"  # a RowNormalization value
MOMENTUM_FORM_KEY: Final = "momentum_form"       # a MomentumForm value

# Fixed when the groups are built; load_state_dict refuses a change.
STRUCTURAL_KEYS: Final = (
    ROUTE_KEY,
    FRACTION_KEY,
    NUM_HEADS_KEY,
    NEWTON_SCHULZ_KEY,
    ROW_NORMALIZATION_KEY,
    MOMENTUM_FORM_KEY,
)

# Per-parameter state keys.
MOMENTUM_STATE: Final = "momentum"
VARIANCE_STATE: Final = "variance"
EXP_AVG_STATE: Final = "exp_avg"
EXP_AVG_SQ_STATE: Final = "exp_avg_sq"
# Not "step": torch's loader would move a "step" entry to the CPU, and this
# counter must stay a device scalar so that a step never synchronizes.
ADAMW_STEP_STATE: Final = "adamw_step"

__all__ = [
    "ADAMW_STEP_STATE",
    "EXP_AVG_SQ_STATE",
    "EXP_AVG_STATE",
    "FRACTION_KEY",
    "MOMENTUM_FORM_KEY",
    "MOMENTUM_KEY",
    "MOMENTUM_STATE",
    "MUON_BETA2_KEY",
    "NEWTON_SCHULZ_KEY",
    "NUM_HEADS_KEY",
    "ROUTE_KEY",
    "ROW_NORMALIZATION_KEY",
    "STRUCTURAL_KEYS",
    "VARIANCE_STATE",
    "ParamState",
]
