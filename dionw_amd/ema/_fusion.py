"""The EMA tracker a running optimizer step may fuse shadow updates with.

Set by ``Dion.step`` around its passes when the integrated EMA is due; read by
the matrix and AdamW passes (through a context variable, so that the
``step_run`` / ``adamw_step`` signatures stay the reference's).
"""

from __future__ import annotations

from contextvars import ContextVar
from typing import TYPE_CHECKING

if TYPE_CHECKING:
    from dionw_amd.ema.tracker import OptimizerIntegratedEMA

__all__ = ["ACTIVE_EMA"]

ACTIVE_EMA: ContextVar[OptimizerIntegratedEMA | None] = ContextVar("dionw_active_ema", default=None)
