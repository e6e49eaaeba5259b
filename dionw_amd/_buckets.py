"""Matrix state packed by block shape, one allocation per shape.

The matrix parameters of a param group split into blocks (``matrix_blocks``:
a head split divides the rows, trailing dims flatten into columns). Blocks of
one ``(rows, cols)`` on one device form a bucket, whose float32 momentum
``[N, rows, cols]`` and NorMuon variance ``[N, rows, 1]`` are single
zero-initialized tensors in HBM; ``optimizer.state[p]`` holds views of them, so
a step walks a whole run of a bucket as one contiguous array (the HIP passes
take it as ``[blocks * rows, cols]``) and ``torch.save`` keeps one storage per
bucket, as the reference's checkpoints do (_buckets.py:43-191). State that is
already present (a loaded checkpoint, an earlier packing) is copied in.

``newton_schulz_fn`` is looked up here each time buckets are packed, so a
caller can replace the orthogonalization by patching this module.
"""

from __future__ import annotations

import math
from collections.abc import Sequence
from dataclasses import dataclass
from typing import Any

import torch
from torch import Tensor, nn

from dionw_amd._groups import GroupSpec, matrix_blocks
from dionw_amd._keys import MOMENTUM_STATE, VARIANCE_STATE, ParamState
from dionw_amd.newton_schulz import Orthogonalize, newton_schulz_fn
from dionw_amd.routing import RouteKind

__all__ = ["Bucket", "block_shape", "pack_buckets"]

# The reference's name for the block split of a parameter.
block_shape = matrix_blocks


@dataclass(eq=False)
class Bucket:
    """Same-shape blocks of one param group and their packed state.

    Attributes:
        group_index: Position of the param group the blocks belong to.
        orthogonalize: The group's orthogonalization.
        params: Parameters with blocks in the bucket, ordered as in their group.
        offsets: First block of each parameter, then the block count.
        rows, cols: Shape of one block.
        selected_rows: Rows updated per step, ``min(rows, ceil(fraction * rows))``.
        momentum: ``[N, rows, cols]`` float32.
        variance: ``[N, rows, 1]`` float32.
    """

    group_index: int
    orthogonalize: Orthogonalize
    params: list[nn.Parameter]
    offsets: list[int]
    rows: int
    cols: int
    selected_rows: int
    momentum: Tensor
    variance: Tensor

    @property
    def blocks_per_param(self) -> int:
        """Blocks of each parameter (the same for all parameters of a bucket)."""
        return self.offsets[1] - self.offsets[0]

    def param_blocks(self, position: int) -> slice:
        """The blocks of the parameter at ``position``."""
        return slice(self.offsets[position], self.offsets[position + 1])

    def run_blocks(self, positions: Sequence[int]) -> slice:
        """The blocks of the consecutive parameters ``positions``."""
        return slice(self.offsets[positions[0]], self.offsets[positions[-1] + 1])

    def adopt(self, state: ParamState) -> None:
        """Point each parameter's momentum and variance entries at views of the
        bucket, copying in whatever values the entries held."""
        for position, param in enumerate(self.params):
            blocks = self.param_blocks(position)
            entry = state[param]
            views = {MOMENTUM_STATE: self.momentum[blocks].view(param.shape),
                     VARIANCE_STATE: self.variance[blocks].view(param.shape[0], 1)}
            for key, view in views.items():
                held = entry.get(key)
                if held is not None:
                    view.copy_(held)
                entry[key] = view


def pack_buckets(param_groups: Sequence[dict[str, Any]], state: ParamState) -> list[Bucket]:
    """Buckets of every matrix group, in group order and, within a group, in the
    order each block shape first appears.

    Raises:
        ValueError: If a head split does not divide a parameter's rows.
    """
    members: dict[tuple[int, int, int, torch.device], list[nn.Parameter]] = {}
    specs: dict[int, GroupSpec] = {}
    for index, group in enumerate(param_groups):
        spec = GroupSpec.of(group)
        if spec.kind is not RouteKind.MATRIX:
            continue
        specs[index] = spec
        for param in group["params"]:
            _, rows, cols = matrix_blocks(param, spec.num_heads)
            members.setdefault((index, rows, cols, param.device), []).append(param)
    kinds = {index: newton_schulz_fn(spec.newton_schulz) for index, spec in specs.items()}
    buckets = []
    for (index, rows, cols, device), params in members.items():
        spec = specs[index]
        offsets = [0]
        for param in params:
            offsets.append(offsets[-1] + matrix_blocks(param, spec.num_heads)[0])
        bucket = Bucket(
            group_index=index,
            orthogonalize=kinds[index],
            params=params,
            offsets=offsets,
            rows=rows,
            cols=cols,
            selected_rows=min(rows, math.ceil(spec.fraction * rows)),
            momentum=torch.zeros(offsets[-1], rows, cols, device=device),
            variance=torch.zeros(offsets[-1], rows, 1, device=device),
        )
        bucket.adopt(state)
        buckets.append(bucket)
    return buckets
