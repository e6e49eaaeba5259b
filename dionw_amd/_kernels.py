"""Per-tensor entry points with the reference's kernel-function signatures.

``accumulate_row_l1`` / ``accumulate_copy_decay`` replace
src/dionw/_momentum_kernels.py:89-133 and ``ns_line_1`` / ``ns_line_2``
replace src/dionw/_symmetric_kernels.py:252-312, on the HIP library. The
optimizer itself calls the run-level entry points (one launch per bucket run);
these serve callers and tests that use the reference's per-tensor interface.
"""

from __future__ import annotations

import torch
from torch import Tensor

from dionw_amd import _lib, _workspace

__all__ = ["accumulate_copy_decay", "accumulate_row_l1", "gemm_nt", "ns_line_1", "ns_line_2"]


def _check(grad: Tensor, momentum: Tensor) -> None:
    if not (grad.is_contiguous() and momentum.is_contiguous()):
        raise ValueError("the fused momentum kernels need contiguous tensors")
    if momentum.dtype != torch.float32 or grad.numel() != momentum.numel():
        raise ValueError("the fused momentum kernels need float32 momentum of the grad's size")
    if grad.dtype != torch.float32:
        raise ValueError("the HIP momentum kernels take float32 gradients")


def accumulate_row_l1(grad: Tensor, momentum: Tensor, scores: Tensor, cols: int) -> None:
    """``momentum += grad``; ``scores[i]`` = l1 norm of momentum row ``i``.

    Raises:
        ValueError: For non-contiguous tensors or a non-float32 momentum.
    """
    _check(grad, momentum)
    rows = momentum.numel() // cols
    if not scores.is_contiguous() or scores.numel() < rows:
        raise ValueError("scores must be contiguous with one element per row")
    rowsq = _workspace.buffer(momentum.device, "l1_rowsq", (rows,), torch.float32)
    _lib.call("dionw_accumulate_scores", _lib.ptr_array([grad]), 1, rows, cols,
              momentum.data_ptr(), scores.data_ptr(), rowsq.data_ptr(),
              _lib.stream_handle(momentum.device))


def accumulate_copy_decay(
    grad: Tensor, momentum: Tensor, out: Tensor, decay: float, *, nesterov: bool
) -> None:
    """``momentum = decay * (momentum + grad)``; ``out`` = the Newton-Schulz input.

    ``out`` is ``momentum + grad`` before the decay, or with ``nesterov``
    ``grad`` plus the decayed momentum.

    Raises:
        ValueError: For non-contiguous tensors or a non-float32 momentum.
    """
    _check(grad, momentum)
    if not out.is_contiguous() or out.numel() != momentum.numel() or out.dtype != torch.float32:
        raise ValueError("out must be a contiguous float32 tensor of the momentum's size")
    numel = momentum.numel()
    if numel == 0:
        return
    dummy = _workspace.buffer(momentum.device, "copy_decay_den", (1,), torch.float32)
    _lib.call("dionw_prepare_ns_input", _lib.ptr_array([grad]), 1, momentum.data_ptr(), None,
              dummy.data_ptr(), 1, 1, numel, 1, 1, numel, float(decay), int(nesterov), 1,
              _lib.F32, out.data_ptr(), None, _lib.stream_handle(momentum.device))


def gemm_nt(
    a: Tensor,
    b: Tensor,
    *,
    d: Tensor | None = None,
    alpha: float = 1.0,
    beta: float = 0.0,
    out: Tensor | None = None,
    out_t: Tensor | None = None,
    symmetric: bool = False,
) -> Tensor | None:
    """Batched ``alpha * a @ b.mT + beta * d`` (float16 or bfloat16, fp32 accumulation).

    ``a`` is ``[..., m, k]``, ``b`` ``[..., n, k]``; ``out`` receives the
    ``[..., m, n]`` result and ``out_t`` (optional) its transpose. With
    ``symmetric`` only the upper tiles are computed and mirrored.
    """
    squeeze = a.ndim == 2
    a3, b3 = (a[None], b[None]) if squeeze else (a, b)
    batch, m, k = (int(x) for x in a3.shape)
    n = int(b3.shape[-2])
    if out is None and out_t is None:
        out = torch.empty(*a.shape[:-1], n, device=a.device, dtype=a.dtype)
    o3 = None if out is None else (out[None] if squeeze else out)
    t3 = None if out_t is None else (out_t[None] if squeeze else out_t)
    d3 = None if d is None else (d[None] if squeeze else d)
    for t in (a3, b3, o3, t3, d3):
        if t is not None and (t.stride(-1) != 1 or t.dtype != a.dtype):
            raise ValueError("gemm_nt: operands must share a 16-bit dtype with unit column stride")

    def strides(t: Tensor | None) -> tuple[int | None, int, int]:
        if t is None:
            return None, 0, 0
        return t.data_ptr(), t.stride(-2), (t.stride(0) if t.shape[0] > 1 else 0)

    pa, lda, sa = strides(a3)
    pb, ldb, sb = strides(b3)
    pd, ldd, sd = strides(d3)
    pc, ldc, sc = strides(o3)
    pt, ldt, st = strides(t3)
    _lib.call("dionw_gemm_nt", _lib.elem_code(a.dtype), batch, m, n, k, pa, lda, sa, pb, ldb, sb,
              pd, ldd, sd, float(alpha), float(beta), pc, ldc, sc, pt, ldt, st, int(symmetric),
              _lib.stream_handle(a.device))
    return out


def _symmetric_output(a: Tensor, out: Tensor | None) -> Tensor:
    if a.ndim not in (2, 3):
        raise ValueError(f"Input tensor must be 2D or 3D, but got {a.ndim}D tensor.")
    rows = a.size(-2)
    if out is None:
        return torch.empty((*a.shape[:-1], rows), device=a.device, dtype=a.dtype)
    if out.shape[-2:] != (rows, rows):
        raise ValueError(f"Output must be [..., {rows}, {rows}], got {out.shape}")
    return out


def ns_line_1(a: Tensor, *, out: Tensor | None = None) -> Tensor:
    """``a @ a.mT`` for a 2-D or batched 3-D 16-bit ``a``, computing half the tiles."""
    out = _symmetric_output(a, out)
    gemm_nt(a, a, out=out, symmetric=True)
    return out


def ns_line_2(a: Tensor, alpha: float, beta: float, *, out: Tensor | None = None) -> Tensor:
    """``alpha * a @ a.mT + beta * a`` for a symmetric square (batched) 16-bit ``a``."""
    rows, cols = a.shape[-2:]
    if rows != cols:
        raise ValueError(f"Input must be symmetric square matrix, but got shape {a.shape}")
    out = _symmetric_output(a, out)
    gemm_nt(a, a, d=a, alpha=alpha, beta=beta, out=out, symmetric=True)
    return out
