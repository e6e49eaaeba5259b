"""Bucketed matrix state: same-shape blocks of a group stored contiguously.

Reference: src/dionw/_buckets.py:43-191. Every bucket owns one float32
momentum ``[N, rows, cols]`` and one variance ``[N, rows, 1]`` for its ``N``
blocks, zero-initialized; ``optimizer.state[p]`` holds views into them, so a
step never stacks parameters and ``torch.save`` keeps the sharing. Blocks are
grouped by ``(rows, cols, device)`` in parameter order. ``newton_schulz_fn`` is
looked up at bucket build time through this module, so tests can replace it.
"""

from __future__ import annotations

import contextlib
import math
from collections.abc import Iterator, Sequence
from dataclasses import dataclass
from typing import Any

import torch
from torch import Tensor, nn

from dionw_amd._keys import (
    FRACTION_KEY,
    MOMENTUM_STATE,
    NEWTON_SCHULZ_KEY,
    NUM_HEADS_KEY,
    ROUTE_KEY,
    VARIANCE_STATE,
    ParamState,
)
from dionw_amd.newton_schulz import NewtonSchulz, Orthogonalize, newton_schulz_fn
from dionw_amd.routing import RouteKind

__all__ = ["Bucket", "block_shape", "build_buckets", "raised_recompile_limits"]


@dataclass
class Bucket:
    """Same-shape blocks of one matrix group.

    Attributes:
        group_index: Index of the owning param group.
        orthogonalize: The group's Newton-Schulz function.
        params: The bucket's parameters, in group order.
        slices: Each parameter's range of blocks.
        rows, cols: Shape of one block.
        selected_rows: Rows updated per step, ``min(rows, ceil(fraction * rows))``.
        momentum: ``[N, rows, cols]`` float32 momentum.
        variance: ``[N, rows, 1]`` float32 NorMuon row variance.
        step_scale: 0-d float32 device tensor kept for layout compatibility
            (the kernels take the signed step by value).
    """

    group_index: int
    orthogonalize: Orthogonalize
    params: list[nn.Parameter]
    slices: list[slice]
    rows: int
    cols: int
    selected_rows: int
    momentum: Tensor
    variance: Tensor
    step_scale: Tensor

    def run_blocks(self, positions: Sequence[int]) -> slice:
        """The blocks of consecutive parameters ``positions``."""
        return slice(self.slices[positions[0]].start, self.slices[positions[-1]].stop)

    @property
    def blocks_per_param(self) -> int:
        """Blocks of each parameter (every parameter of a bucket has as many)."""
        return self.slices[0].stop - self.slices[0].start


def block_shape(param: Tensor, num_heads: int | None) -> tuple[int, int, int]:
    """``(blocks, rows, cols)`` of a matrix parameter: trailing dims flatten into
    columns and a head split divides the rows.

    Raises:
        ValueError: If ``num_heads`` does not divide the rows.
    """
    rows = int(param.shape[0])
    cols = math.prod(int(d) for d in param.shape[1:])
    if num_heads is None:
        return 1, rows, cols
    if rows % num_heads:
        raise ValueError(f"num_heads={num_heads} does not divide {rows} rows")
    return num_heads, rows // num_heads, cols


@contextlib.contextmanager
def raised_recompile_limits() -> Iterator[None]:
    """Compatibility no-op: the HIP path compiles nothing at run time."""
    yield


def build_buckets(param_groups: list[dict[str, Any]], state: ParamState) -> list[Bucket]:
    """Pack every matrix group's state into per-shape buckets (group order).

    Existing momentum and variance entries (a loaded checkpoint or an older
    layout) are copied in; ``state[p]`` then holds views.
    """
    buckets: list[Bucket] = []
    for index, group in enumerate(param_groups):
        if RouteKind(group[ROUTE_KEY]) is not RouteKind.MATRIX:
            continue
        orthogonalize = newton_schulz_fn(NewtonSchulz(group[NEWTON_SCHULZ_KEY]))
        by_shape: dict[tuple[int, int, torch.device], list[nn.Parameter]] = {}
        for param in group["params"]:
            _, rows, cols = block_shape(param, group[NUM_HEADS_KEY])
            by_shape.setdefault((rows, cols, param.device), []).append(param)
        for params in by_shape.values():
            bucket = _new_bucket(index, group, params, orthogonalize)
            _attach_state(bucket, state)
            buckets.append(bucket)
    return buckets


def _new_bucket(
    index: int, group: dict[str, Any], params: list[nn.Parameter], orthogonalize: Orthogonalize
) -> Bucket:
    heads = group[NUM_HEADS_KEY]
    slices: list[slice] = []
    start = 0
    for param in params:
        count = block_shape(param, heads)[0]
        slices.append(slice(start, start + count))
        start += count
    _, rows, cols = block_shape(params[0], heads)
    device = params[0].device
    return Bucket(
        group_index=index,
        orthogonalize=orthogonalize,
        params=params,
        slices=slices,
        rows=rows,
        cols=cols,
        selected_rows=min(rows, math.ceil(float(group[FRACTION_KEY]) * rows)),
        momentum=torch.zeros(start, rows, cols, device=device),
        variance=torch.zeros(start, rows, 1, device=device),
        step_scale=torch.zeros((), device=device),
    )


def _attach_state(bucket: Bucket, state: ParamState) -> None:
    for param, blocks in zip(bucket.params, bucket.slices, strict=True):
        entry = state[param]
        momentum = bucket.momentum[blocks].view(param.shape)
        variance = bucket.variance[blocks].view(param.shape[0], 1)
        if MOMENTUM_STATE in entry:
            momentum.copy_(entry[MOMENTUM_STATE])
            variance.copy_(entry[VARIANCE_STATE])
        entry[MOMENTUM_STATE] = momentum
        entry[VARIANCE_STATE] = variance
