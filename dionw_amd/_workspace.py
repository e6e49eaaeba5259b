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
queue position (names with a ``#i`` suffix), reused from one flush and one step
to the next; the queue drops them all before their total would pass its byte
cap, so they hold at most that cap, or one run's set where a run alone is
larger.
"""

from __future__ import annotations

import math
from collections.abc import Callable

import torch

__all__ = ["buffer", "release", "release_named", "held_bytes", "named_bytes", "share", "tensors"]

_ALIGN = 256
_BUFFERS: dict[tuple[torch.device, int, str], torch.Tensor] = {}


def _resolved(device: torch.device | str) -> torch.device:
    """``device`` with its index filled in: ``cuda`` means the current GPU, so
    that ``cuda`` and ``cuda:0`` name the same buffers when GPU 0 is current."""
    device = torch.device(device)
    if device.type == "cuda" and device.index is None:
        return torch.device("cuda", torch.cuda.current_device())
    return device


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
    device = _resolved(device)
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
    device = None if device is None else _resolved(device)
    for key in [k for k in _BUFFERS if device is None or k[0] == device]:
        _retire(_BUFFERS.pop(key), key[1])


def named_bytes(device: torch.device, stream: int, match: Callable[[str], bool]) -> int:
    """Bytes held by the buffers of ``device`` and ``stream`` whose names ``match``."""
    device = _resolved(device)
    return sum(t.numel() for (dev, st, name), t in _BUFFERS.items()
               if dev == device and st == stream and match(name))


def release_named(device: torch.device, stream: int, match: Callable[[str], bool]) -> None:
    """Drop the buffers of ``device`` and ``stream`` whose names ``match``."""
    device = _resolved(device)
    for key in [k for k in _BUFFERS if k[0] == device and k[1] == stream and match(k[2])]:
        _retire(_BUFFERS.pop(key), key[1])


def held_bytes(device: torch.device | None = None) -> int:
    """Bytes held by the scratch buffers (of ``device``, or all)."""
    device = None if device is None else _resolved(device)
    unique = {t.data_ptr(): t.numel() for k, t in _BUFFERS.items()
              if device is None or k[0] == device}
    return sum(unique.values())


def share(device: torch.device, source: int, target: int) -> None:
    """Let work on stream ``target`` use the buffers of stream ``source``
    (names it has none of yet). For a stream that only records launches made
    in stream order with ``source``'s, such as a graph capture stream whose
    replays run on ``source``: the recorded launches then use the same scratch
    as eager steps instead of a second copy."""
    device = _resolved(device)
    for (dev, stream, name), store in list(_BUFFERS.items()):
        if dev == device and stream == source:
            _BUFFERS.setdefault((dev, target, name), store)


def tensors(device: torch.device | None = None) -> list[torch.Tensor]:
    """The scratch buffers held now (of ``device``, or all), e.g. to keep them
    alive for launches recorded in a graph."""
    device = None if device is None else _resolved(device)
    return [t for k, t in _BUFFERS.items() if device is None or k[0] == device]
