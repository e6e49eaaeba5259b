"""Scratch buffers of the HIP passes, one named set per device and stream.

A step's kernels run in order on one stream, so one set of named buffers per
(device, stream) serves every run; a buffer grows (never shrinks) to the
largest request. Work issued on two streams never shares a buffer, and a
buffer that is dropped or regrown is recorded on its stream first, so the
caching allocator does not hand its memory to other work before the kernels
that use it have run. The HIP library itself never allocates: everything it
touches comes from here or from the optimizer state.

``release`` drops the buffers (the optimizer calls it when its packing
changes); they are recreated on demand. A queued step keeps one buffer set per
queued run (names with a ``#i`` suffix) until its grouped orthogonalization
has run, so the peak is the sum over the runs of one flush: at most the queue's
byte cap plus the largest run.
"""

from __future__ import annotations

import math

import torch

__all__ = ["buffer", "release", "held_bytes"]

_ALIGN = 256
_BUFFERS: dict[tuple[torch.device, int, str], torch.Tensor] = {}


def _stream_of(device: torch.device) -> int:
    if device.type != "cuda":
        return 0
    return torch.cuda.current_stream(device).cuda_stream


def _retire(store: torch.Tensor, stream: int) -> None:
    """Tell the allocator that ``store`` is in use on ``stream`` until the work
    queued there so far has run."""
    if store.is_cuda:
        store.record_stream(torch.cuda.ExternalStream(stream, device=store.device))


def buffer(device: torch.device, name: str, shape: tuple[int, ...], dtype: torch.dtype,
           stream: int | None = None) -> torch.Tensor:
    """A ``shape`` view of the named scratch buffer of ``device`` and ``stream``
    (torch's current stream on ``device`` when None); uninitialized."""
    device = torch.device(device)
    stream = _stream_of(device) if stream is None else stream
    numel = math.prod(shape)
    nbytes = max(numel * torch.empty((), dtype=dtype).element_size(), 1)
    key = (device, stream, name)
    store = _BUFFERS.get(key)
    if store is None or store.numel() < nbytes:
        if store is not None:
            _retire(store, stream)
        store = torch.empty(((nbytes + _ALIGN - 1) // _ALIGN) * _ALIGN, dtype=torch.uint8,
                            device=device)
        _BUFFERS[key] = store
    return store[:nbytes].view(dtype)[:numel].view(shape)


def release(device: torch.device | None = None) -> None:
    """Drop the scratch buffers (of ``device``, or all)."""
    for key in [k for k in _BUFFERS if device is None or k[0] == torch.device(device)]:
        _retire(_BUFFERS.pop(key), key[1])


def held_bytes(device: torch.device | None = None) -> int:
    """Bytes held by the scratch buffers (of ``device``, or all)."""
    return sum(t.numel() for k, t in _BUFFERS.items()
               if device is None or k[0] == torch.device(device))
