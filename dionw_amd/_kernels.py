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

_PRODUCT_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def _check(grad: Tensor, momentum: Tensor) -> Tensor:
    """The gradient as the kernels read it: contiguous float32.

    Any float gradient is accepted, as in the reference (its kernels load and
    upcast): float16 and bfloat16 convert to float32 exactly.
    """
    if not (grad.is_contiguous() and momentum.is_contiguous()):
        raise ValueError("the momentum kernels take contiguous tensors only")
    if momentum.dtype != torch.float32 or grad.numel() != momentum.numel():
        raise ValueError("the momentum kernels take a float32 momentum with as many elements as the gradient")
    if not grad.is_floating_point():
        raise ValueError(f"the momentum kernels take a float gradient, not {grad.dtype}")
    if grad.device != momentum.device:
        raise ValueError("grad and momentum must be on the same device")
    return grad if grad.dtype == torch.float32 else grad.to(torch.float32)


def accumulate_row_l1(grad: Tensor, momentum: Tensor, scores: Tensor, cols: int) -> None:
    """Adds ``grad`` into ``momentum`` and writes each row's sum of absolute
    values into ``scores``.

    Raises:
        ValueError: For non-contiguous tensors, a non-float32 momentum or a
            non-float gradient.
    """
    grad = _check(grad, momentum)
    rows = momentum.numel() // cols
    if not scores.is_contiguous() or scores.numel() < rows or scores.dtype != torch.float32:
        raise ValueError("scores must be contiguous float32 with one element per row")
    rowsq = _workspace.buffer(momentum.device, "l1_rowsq", (rows,), torch.float32)
    _lib.call("dionw_accumulate_scores", _lib.ptr_array([grad]), 1, rows, cols,
              momentum.data_ptr(), scores.data_ptr(), rowsq.data_ptr(), _lib.F32,
              _lib.stream_handle(momentum.device))


def accumulate_copy_decay(
    grad: Tensor, momentum: Tensor, out: Tensor, decay: float, *, nesterov: bool
) -> None:
    """Writes the Newton-Schulz input to ``out`` and leaves the decayed sum
    ``decay * (momentum + grad)`` in ``momentum``.

    ``out`` is ``momentum + grad`` before the decay, or with ``nesterov``
    ``grad`` plus the decayed momentum.

    Raises:
        ValueError: For non-contiguous tensors, a non-float32 momentum or a
            non-float gradient.
    """
    grad = _check(grad, momentum)
    if not out.is_contiguous() or out.numel() != momentum.numel() or out.dtype != torch.float32:
        raise ValueError("out must be a contiguous float32 tensor of the momentum's size")
    numel = momentum.numel()
    if numel == 0:
        return
    dummy = _workspace.buffer(momentum.device, "copy_decay_den", (1,), torch.float32)
    _lib.call("dionw_prepare_ns_input", _lib.ptr_array([grad]), 1, momentum.data_ptr(), None,
              dummy.data_ptr(), 1, 1, numel, 1, 1, numel, float(decay), int(nesterov), 1,
              _lib.F32, out.data_ptr(), None, _lib.stream_handle(momentum.device))


def _as3(t: Tensor | None, squeeze: bool) -> Tensor | None:
    return None if t is None else (t[None] if squeeze else t)


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
    """Batched ``alpha * a @ b.mT + beta * d`` (fp32 accumulation).

    ``a`` is ``[..., m, k]``, ``b`` ``[..., n, k]`` (2-D, or 3-D with one batch
    dimension), float16, bfloat16 or float32; ``out`` receives the
    ``[..., m, n]`` result and ``out_t`` (optional) its transpose. With
    ``symmetric`` only the upper tiles are computed and mirrored.

    Raises:
        ValueError: For operands that disagree in shape, batch, dtype or device,
            or without a unit column stride.
    """
    if a.ndim not in (2, 3) or b.ndim != a.ndim:
        raise ValueError(f"gemm_nt: a and b must both be 2-D or 3-D, got {a.ndim}-D and {b.ndim}-D")
    if a.dtype not in _PRODUCT_DTYPES:
        raise ValueError(f"gemm_nt: unsupported dtype {a.dtype}")
    squeeze = a.ndim == 2
    a3, b3 = _as3(a, squeeze), _as3(b, squeeze)
    batch, m, k = (int(x) for x in a3.shape)
    n = int(b3.shape[-2])
    if int(b3.shape[0]) != batch or int(b3.shape[-1]) != k:
        raise ValueError(f"gemm_nt: b {tuple(b.shape)} does not match a {tuple(a.shape)}")
    if out is None and out_t is None:
        out = torch.empty(*a.shape[:-1], n, device=a.device, dtype=a.dtype)
    o3, t3, d3 = _as3(out, squeeze), _as3(out_t, squeeze), _as3(d, squeeze)
    expect = {"out": (o3, (batch, m, n)), "out_t": (t3, (batch, n, m)), "d": (d3, (batch, m, n))}
    for name, (t, shape) in expect.items():
        if t is not None and tuple(t.shape) != shape:
            got = out if name == "out" else out_t if name == "out_t" else d
            raise ValueError(f"gemm_nt: {name} must be {shape[1:] if squeeze else shape}, "
                             f"got {tuple(got.shape)}")
    for t in (a3, b3, o3, t3, d3):
        if t is None:
            continue
        if t.dtype != a.dtype or t.device != a.device:
            raise ValueError("gemm_nt: operands must share a's dtype and device")
        if t.stride(-1) != 1:
            raise ValueError("gemm_nt: operands need a unit column stride")
    if symmetric and (m != n or out is None or out_t is not None):
        raise ValueError("gemm_nt: a symmetric product needs m == n and out only")

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


def _square_out(a: Tensor, out: Tensor | None) -> Tensor:
    if a.ndim not in (2, 3):
        raise ValueError(f"expected a 2-D matrix or a 3-D batch, got {a.ndim} dimensions")
    rows = a.size(-2)
    if out is None:
        return torch.empty((*a.shape[:-1], rows), device=a.device, dtype=a.dtype)
    if tuple(out.shape) != (*a.shape[:-1], rows):
        raise ValueError(f"out has shape {tuple(out.shape)}; the product needs "
                         f"{(*a.shape[:-1], rows)}")
    return out


def ns_line_1(a: Tensor, *, out: Tensor | None = None) -> Tensor:
    """``a @ a.mT`` for a 2-D or batched 3-D ``a``, computing half the tiles.

    float16 and bfloat16 run on the 16-bit MFMA kernels (float32 accumulation,
    output in a's dtype); float32 on the float32 MFMA (the reference's "ieee"
    precision for float32 inputs).
    """
    out = _square_out(a, out)
    gemm_nt(a, a, out=out, symmetric=True)
    return out


def ns_line_2(a: Tensor, alpha: float, beta: float, *, out: Tensor | None = None) -> Tensor:
    """``alpha * a @ a.mT + beta * a`` for a symmetric square (batched) ``a``,
    computing half the tiles (dtypes as ``ns_line_1``)."""
    rows, cols = a.shape[-2:]
    if rows != cols:
        raise ValueError(f"expected square (symmetric) matrices, got shape {tuple(a.shape)}")
    out = _square_out(a, out)
    gemm_nt(a, a, d=a, alpha=alpha, beta=beta, out=out, symmetric=True)
    return out
