"""Memory-layout predicates for the element-wise multi-tensor kernels."""

from __future__ import annotations

from torch import Tensor

__all__ = ["dense", "same_dense_layout"]


def dense(tensor: Tensor) -> bool:
    """Whether the elements tile one contiguous storage span without overlap
    (row-major, channels-last or any other permutation of a contiguous layout)."""
    expected = 1
    for size, stride in sorted(zip(tensor.shape, tensor.stride()), key=lambda d: d[1]):
        if size == 1:
            continue
        if stride != expected:
            return False
        expected *= size
    return True


def same_dense_layout(a: Tensor, b: Tensor) -> bool:
    """Both dense with identical shape and strides (element i of one storage
    pairs with element i of the other)."""
    return a.shape == b.shape and a.stride() == b.stride() and dense(a) and dense(b)
