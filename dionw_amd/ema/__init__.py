"""An exponential moving average of the parameters kept by the optimizer (GPU or CPU shadows).

Reference: src/dionw/ema/__init__.py. Shadows live in ``optimizer.state[p]``
(``ema_shadow``, float32); the schedule position is the top-level
``_ema_step_count`` entry. The EMA updates after each due optimizer step with
decay ``decay ** n`` (``update_every_n_steps = n``); every update is a lerp,
so a constant parameter keeps a bit-exact shadow.
"""

from dionw_amd.ema._keys import EMA_STEP_COUNT_KEY
from dionw_amd.ema.config import EMAConfig, EMADevice, EMASchedule, ProfileRegion, no_profile
from dionw_amd.ema.mixin import IntegratedEMAOptimizer
from dionw_amd.ema.tracker import OptimizerIntegratedEMA

__all__ = [
    "EMA_STEP_COUNT_KEY",
    "EMAConfig",
    "EMADevice",
    "EMASchedule",
    "IntegratedEMAOptimizer",
    "OptimizerIntegratedEMA",
    "ProfileRegion",
    "no_profile",
]
