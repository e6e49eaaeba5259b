"""One ``Dion.step`` captured as a HIP graph and replayed (opt-in).

A step is 40-80 launches issued from Python; replaying them as one graph
removes the host's part of the step (the Python dispatch and the launch
calls) and the gaps between launches. The graph repeats exactly the step it
recorded:

- the same gradient tensors: keep gradients in fixed storage (for example
  ``zero_grad(set_to_none=False)``, or copy new gradients into the recorded
  ``.grad`` tensors before each replay);
- the same hyperparameters: the learning rate and the other group options
  are baked into the launches (capture again after changing them);
- the same packing: capture again after ``add_param_group`` or
  ``load_state_dict``;
- no EMA: its schedule runs on the host each step (``Dion.step`` refuses to
  be captured with one).

AdamW's step counters live on the device, so bias corrections advance with
every replay as they do with eager steps; replays produce the eager steps'
results bit for bit.

The capture records on a stream of its own; the step's scratch buffers are
those of the stream the graph was captured from (``_workspace.share``), and
the graph holds them, so eager steps and replays issued on that stream share
one set.
"""

from __future__ import annotations

import torch

from dionw_amd import _workspace
from dionw_amd.optimizer import Dion

__all__ = ["StepGraph"]


class StepGraph:
    """``optimizer.step()`` recorded once, replayed with ``replay()``.

    Captured on the current stream's device; ``replay`` launches the graph on
    the stream current at the call, like an eager step.
    """

    def __init__(self, optimizer: Dion) -> None:
        """Pack the optimizer's state if needed, then record one step.

        Recording runs nothing: parameters and state are unchanged until the
        first replay.

        Raises:
            RuntimeError: For an optimizer with an EMA, or without a GPU.
            TypeError: For an optimizer that is not a ``Dion``.
        """
        if not isinstance(optimizer, Dion):
            raise TypeError(f"StepGraph records a Dion step, not {type(optimizer).__name__}")
        if not torch.cuda.is_available():
            raise RuntimeError("StepGraph needs a GPU")
        if optimizer.ema is not None:
            raise RuntimeError("StepGraph: the EMA's schedule runs on the host each step and "
                               "cannot be replayed; record a Dion without an EMA")
        params = [p for g in optimizer.param_groups for p in g["params"]]
        device = params[0].device if params else torch.device("cuda",
                                                              torch.cuda.current_device())
        # Packing zeroes and copies state: do it now, outside the recording.
        optimizer._buckets()
        current = torch.cuda.current_stream(device)
        capture = torch.cuda.Stream(device)
        _workspace.share(device, current.cuda_stream, capture.cuda_stream)
        capture.wait_stream(current)
        self.optimizer = optimizer
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=capture):
            optimizer.step()
        current.wait_stream(capture)
        # Buffers the recorded launches address: held for the graph's lifetime
        # (a release or regrowth of the workspace must not free them).
        self._held = _workspace.tensors(device)

    def replay(self) -> None:
        """One step: the recorded launches on the current stream."""
        self.graph.replay()
