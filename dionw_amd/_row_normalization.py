"""The row-normalization seam of a matrix step: NorMuon or none, times the step.

Reference: src/dionw/_row_normalization.py:18-60 (``finish`` and
``normalize_rows``), with the same names, arguments and results. The
optimizer's own step does not come through here: it fuses the row statistics
and the scaled update into the weight update (``dionw_normuon_stats`` then
``dionw_apply_update`` on the weights), so the float32 step is never written to
HBM. These functions serve callers and tests that use the reference's
interface, and produce the step that fused path adds to the weights.

Both run on the HIP library: ``dionw_normuon_stats`` computes each row's
``v' = lerp(v, mean(O^2), 1 - beta2)``, its divisor ``sqrt(v') + 1e-8`` and
each block's ``||O||_F / max(||O / d||_F, 1e-8) * step``; the step itself is
then ``dionw_apply_update`` on a zeroed float32 buffer with weight decay off,
which stores ``0 + (O / d) * scale``, the very value the fused pass adds to
``W * decay``. Without row normalization the same pass stores
``0 + O * step``, the reference's ``orthogonal.float() * step``.
"""

from __future__ import annotations

from typing import Any, Final

import torch
from torch import Tensor

from dionw_amd import _lib, _workspace
from dionw_amd._keys import MUON_BETA2_KEY, ROW_NORMALIZATION_KEY
from dionw_amd.matrix_update import RowNormalization

__all__ = ["NORMALIZATION_EPS", "finish", "normalize_rows"]

# Added to sqrt(v) and the lower bound of the normalized norm (the kernels'
# literal 1e-8; reference _row_normalization.py:15).
NORMALIZATION_EPS: Final[float] = 1e-8


def _scalar(step: Tensor | float) -> float:
    """The step as the kernels take it: a float32 value (a 0-d tensor is read
    once, as the reference's compiled function reads its 0-d step)."""
    if isinstance(step, Tensor):
        if step.numel() != 1:
            raise ValueError(f"step must be a scalar, got a tensor of shape {tuple(step.shape)}")
        return float(step.detach().to(torch.float32).item())
    return float(torch.tensor(step, dtype=torch.float32))


def _orthogonal(orthogonal: Tensor) -> Tensor:
    if orthogonal.ndim != 3:
        raise ValueError(f"expected a [blocks, k, cols] batch, got {tuple(orthogonal.shape)}")
    if not orthogonal.is_cuda:
        raise ValueError("the HIP row normalization needs GPU tensors")
    if not orthogonal.is_floating_point():
        raise ValueError(f"expected a float batch, got {orthogonal.dtype}")
    # The kernels read bf16, the Newton-Schulz output type; other float types
    # are rounded to it first (the reference reads its bf16 output too).
    return orthogonal.to(torch.bfloat16).contiguous()


def _scaled(orthogonal: Tensor, rowd: Tensor | None, scale: Tensor | None,
            step: float) -> Tensor:
    """``0 + (O / rowd) * scale`` (or ``0 + O * step``) as float32, from the
    weight-update pass run on a zeroed buffer."""
    blocks, k, cols = orthogonal.shape
    out = torch.zeros(blocks, k, cols, device=orthogonal.device, dtype=torch.float32)
    if out.numel() == 0:
        return out
    _lib.call("dionw_apply_update", _lib.ptr_array([out]), 1, blocks, k, cols, k,
              orthogonal.data_ptr(), None, None, None if rowd is None else rowd.data_ptr(),
              None if scale is None else scale.data_ptr(), step, 1.0, 0,
              _lib.stream_handle(out.device))
    return out


def normalize_rows(
    update: Tensor, variance: Tensor, beta2: float, step: Tensor | float
) -> tuple[Tensor, Tensor]:
    """NorMuon row normalization of a ``[blocks, k, cols]`` batch.

    Each row is divided by the root of an EMA of its mean square (``variance``,
    ``[blocks, k, 1]`` float32, is not modified), the block's Frobenius norm is
    restored, and the result is multiplied by ``step``.

    Returns:
        The float32 step ``[blocks, k, cols]`` and the new ``[blocks, k, 1]``
        variance.

    Raises:
        ValueError: For tensors that are not on a GPU or whose shapes disagree.
    """
    orthogonal = _orthogonal(update)
    blocks, k, cols = (int(d) for d in orthogonal.shape)
    if tuple(variance.shape) != (blocks, k, 1) or variance.dtype != torch.float32:
        raise ValueError(f"variance must be float32 [{blocks}, {k}, 1], got "
                         f"{variance.dtype} {tuple(variance.shape)}")
    if variance.device != orthogonal.device:
        raise ValueError("variance and the update must be on the same device")
    new_variance = variance.detach().clone(memory_format=torch.contiguous_format)
    if blocks == 0 or k == 0 or cols == 0:
        return torch.zeros(blocks, k, cols, device=orthogonal.device), new_variance
    scalar = _scalar(step)
    device = orthogonal.device
    rowd = torch.empty(blocks, k, device=device, dtype=torch.float32)
    scale = torch.empty(blocks, device=device, dtype=torch.float32)
    partials = _workspace.buffer(device, "finish_partials", (2 * blocks * k,), torch.float32)
    # Every row is a selected row here (no index table): the variance is the
    # batch's own [blocks, k] rows.
    _lib.call("dionw_normuon_stats", orthogonal.data_ptr(), blocks, k, k, cols, None,
              new_variance.data_ptr(), float(beta2), scalar, rowd.data_ptr(),
              partials.data_ptr(), scale.data_ptr(), _lib.stream_handle(device))
    return _scaled(orthogonal, rowd, scale, scalar), new_variance


def finish(
    orthogonal: Tensor, variance: Tensor, group: dict[str, Any], step: Tensor | float
) -> tuple[Tensor, Tensor | None]:
    """Scale an orthogonalized ``[blocks, k, cols]`` batch into the float32 step.

    Returns:
        The step and, for NorMuon, the new ``[blocks, k, 1]`` variance (None
        without row normalization).

    Raises:
        RuntimeError: For an unhandled ``RowNormalization``.
    """
    match RowNormalization(group[ROW_NORMALIZATION_KEY]):
        case RowNormalization.NORMUON:
            return normalize_rows(orthogonal, variance, float(group[MUON_BETA2_KEY]), step)
        case RowNormalization.NONE:
            return _scaled(_orthogonal(orthogonal), None, None, _scalar(step)), None
        case _ as unreachable:
            raise RuntimeError(f"Unhandled RowNormalization: {unreachable}")
