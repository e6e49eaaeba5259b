"""EMA shadow arithmetic: ``lerp`` toward the live weights.

Reference: src/dionw/ema/_update.py:17-70. Every GPU shadow updates through the
multi-tensor HIP kernel (one launch per 48 tensors, torch's lerp arithmetic, so
a constant parameter keeps a bit-exact shadow): a source of another dtype or
layout is first copied into a float32 tensor laid out like the shadow, and a
shadow that is not dense is updated in a dense copy that is copied back, a
bounded chunk of such pairs at a time. CPU shadows (CPU EMA) are updated on
the host with torch's CPU lerp, as the reference's CPU EMA does.
"""

from __future__ import annotations

from typing import Final

import torch
from torch import Tensor

from dionw_amd import _lib
from dionw_amd._layout import dense, same_dense_layout

__all__ = ["FP32", "ema_update_", "foreach_ema_copy_", "foreach_ema_update_"]

FP32: Final[torch.dtype] = torch.float32
_STAGING_CHUNK_NUMEL: Final[int] = 1 << 24


def ema_update_(shadow: Tensor, source: Tensor, *, decay: float) -> None:
    """``shadow = lerp(shadow, source, 1 - decay)`` in place (any device)."""
    shadow.lerp_(source, 1.0 - decay)


def _hip_lerp(shadows: list[Tensor], sources: list[Tensor], weight: float, copy: bool) -> None:
    if not shadows:
        return
    _lib.call(
        "dionw_ema_update",
        _lib.ptr_array(shadows),
        _lib.ptr_array(sources),
        _lib.int64_array([s.numel() for s in shadows]),
        len(shadows),
        float(weight),
        int(copy),
        _lib.stream_handle(shadows[0].device),
    )


def _kernel_ready(shadow: Tensor, source: Tensor) -> bool:
    # The kernel is element-wise over the storage: any dense layout works as
    # long as both tensors share it (a channels-last weight and its shadow).
    return shadow.is_cuda and source.is_cuda and source.dtype == FP32 and same_dense_layout(shadow, source)


@torch.no_grad()
def foreach_ema_update_(shadows: list[Tensor], sources: list[Tensor], *, decay: float) -> None:
    """``ema_update_`` over lists of shadows and sources.

    Raises:
        TypeError: If a shadow is not float32.
        ValueError: If there are more shadows than sources or the other way round.
    """
    if any(shadow.dtype != FP32 for shadow in shadows):
        raise TypeError("every EMA shadow is kept in float32")
    if len(shadows) != len(sources):
        raise ValueError("shadows and sources differ in length")
    weight = 1.0 - decay
    direct_s: list[Tensor] = []
    direct_p: list[Tensor] = []
    staged: list[tuple[Tensor, Tensor]] = []
    for shadow, source in zip(shadows, sources, strict=True):
        if not shadow.is_cuda:
            ema_update_(shadow, source.to(shadow.device, FP32), decay=decay)
        elif shadow.shape != source.shape:
            raise ValueError(f"EMA shadow {tuple(shadow.shape)} and source "
                             f"{tuple(source.shape)} differ in shape")
        elif _kernel_ready(shadow, source):
            direct_s.append(shadow)
            direct_p.append(source)
        else:
            staged.append((shadow, source))
    _hip_lerp(direct_s, direct_p, weight, copy=False)
    start = 0
    while start < len(staged):
        stop, numel = start + 1, staged[start][1].numel()
        while stop < len(staged) and numel + staged[stop][1].numel() <= _STAGING_CHUNK_NUMEL:
            numel += staged[stop][1].numel()
            stop += 1
        targets = [s if dense(s) else s.contiguous() for s, _ in staged[start:stop]]
        inputs = [torch.empty_like(t).copy_(src) for t, (_, src) in zip(targets, staged[start:stop])]
        _hip_lerp(targets, inputs, weight, copy=False)
        for target, (shadow, _) in zip(targets, staged[start:stop]):
            if target is not shadow:
                shadow.copy_(target)
        start = stop


@torch.no_grad()
def foreach_ema_copy_(shadows: list[Tensor], sources: list[Tensor]) -> None:
    """Copy sources into shadows (the first update of a shadow)."""
    direct_s: list[Tensor] = []
    direct_p: list[Tensor] = []
    for shadow, source in zip(shadows, sources, strict=True):
        if _kernel_ready(shadow, source):
            direct_s.append(shadow)
            direct_p.append(source)
        else:
            shadow.copy_(source)
    _hip_lerp(direct_s, direct_p, 1.0, copy=True)
