"""Names of the EMA's optimizer-state entries (reference: src/dionw/ema/_keys.py:19-33)."""

from __future__ import annotations

from typing import Final

EMA_STEP_COUNT_KEY: Final = "_ema_step_count"  # top-level: schedule position
EMA_KEY_PREFIX: Final = "ema_"                  # every per-parameter EMA entry
EMA_SHADOW: Final = "ema_shadow"                # the float32 shadow
EMA_INITIALIZED: Final = "ema_initialized"      # copied from the live weights yet
EMA_PENDING: Final = "ema_pending"              # a CPU update is queued
EMA_TMP_CPU: Final = "ema_tmp_cpu"              # pinned CPU staging buffer
EMA_EVENT: Final = "ema_event"                  # event of the staged copy
EMA_SCRATCH_KEYS: Final = (EMA_PENDING, EMA_TMP_CPU, EMA_EVENT)  # never saved

__all__ = [
    "EMA_EVENT",
    "EMA_INITIALIZED",
    "EMA_KEY_PREFIX",
    "EMA_PENDING",
    "EMA_SCRATCH_KEYS",
    "EMA_SHADOW",
    "EMA_STEP_COUNT_KEY",
    "EMA_TMP_CPU",
]
