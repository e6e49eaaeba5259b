"""Per-device scratch buffers shared by every bucket run.

Runs execute one after another on the current stream, so one set of named
buffers per device serves them all; a buffer grows (never shrinks) to the
largest request. The HIP library itself never allocates: everything it
touches comes from here or from the optimizer state, through torch's caching
allocator.
"""

from __future__ import annotations

import math

import torch

__all__ = ["buffer"]

_ALIGN = 256
_BUFFERS: dict[tuple[torch.device, str], torch.Tensor] = {}


def buffer(device: torch.device, name: str, shape: tuple[int, ...], dtype: torch.dtype) -> torch.Tensor:
    """A ``shape`` view of the named scratch buffer of ``device`` (uninitialized)."""
    numel = math.prod(shape)
    nbytes = max(numel * torch.empty((), dtype=dtype).element_size(), 1)
    key = (device, name)
    store = _BUFFERS.get(key)
    if store is None or store.numel() < nbytes:
        _BUFFERS.pop(key, None)
        store = torch.empty(((nbytes + _ALIGN - 1) // _ALIGN) * _ALIGN, dtype=torch.uint8,
                            device=device)
        _BUFFERS[key] = store
    return store[:nbytes].view(dtype)[:numel].view(shape)


def release() -> None:
    """Drop every scratch buffer (they are recreated on demand)."""
    _BUFFERS.clear()
