"""dionw_amd: the Dion optimizer step on MI355X (gfx950) HIP kernels.

Drop-in for ``dionw`` (JTriggerFish/dionw): the same public names, param-group
and state keys, so ``import dionw_amd as dionw`` keeps user code unchanged::

    import dionw_amd as dionw

    groups, report = dionw.param_groups(model)
    optimizer = dionw.Dion(groups, lr=3e-4, weight_decay=0.05)
"""

from dionw_amd._keys import (
    FRACTION_KEY,
    MOMENTUM_FORM_KEY,
    NEWTON_SCHULZ_KEY,
    NUM_HEADS_KEY,
    ROUTE_KEY,
    ROW_NORMALIZATION_KEY,
)
from dionw_amd.ema import EMAConfig, EMADevice, EMASchedule, IntegratedEMAOptimizer
from dionw_amd.matrix_update import (
    DION3_UPDATE,
    MUON_UPDATE,
    MatrixUpdate,
    MomentumForm,
    RowNormalization,
)
from dionw_amd.newton_schulz import NewtonSchulz
from dionw_amd.optimizer import Dion
from dionw_amd.param_groups import ParamGroups, param_groups
from dionw_amd.report import RoutedParameter, RouteReason, RoutingReport
from dionw_amd.routing import Route, RouteKind, RouteProvider
# Not in the reference: frees the device scratch the HIP passes keep between steps
# (it grows to the largest run queued; a later step allocates it again).
from dionw_amd._workspace import release as release_workspace  # noqa: F401
# Not in the reference: one step recorded as a HIP graph and replayed.
from dionw_amd.graph import StepGraph  # noqa: F401

__version__ = "0.1.0"

__all__ = [
    "DION3_UPDATE",
    "FRACTION_KEY",
    "MOMENTUM_FORM_KEY",
    "MUON_UPDATE",
    "NEWTON_SCHULZ_KEY",
    "NUM_HEADS_KEY",
    "ROUTE_KEY",
    "ROW_NORMALIZATION_KEY",
    "Dion",
    "EMAConfig",
    "EMADevice",
    "EMASchedule",
    "IntegratedEMAOptimizer",
    "MatrixUpdate",
    "MomentumForm",
    "NewtonSchulz",
    "ParamGroups",
    "Route",
    "RouteKind",
    "RouteProvider",
    "RouteReason",
    "RoutedParameter",
    "RoutingReport",
    "RowNormalization",
    "__version__",
    "param_groups",
]
