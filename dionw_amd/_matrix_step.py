"""The Dion update of a run: consecutive parameters of a bucket that all have gradients.

Reference: src/dionw/_matrix_step.py:104-311. Per block:

1. accumulate ``M += G`` (with each row's l1 score when rows are selected);
2. select the top ``k`` rows and decay them in ``M`` (error feedback), or, when
   every row is updated, ``M = mu (M + G)`` with the heavy-ball or Nesterov
   input;
3. orthogonalize the selected (or all) rows;
4. NorMuon row normalization, or none, times the signed step;
5. decoupled weight decay on every row, then the update on the selected rows.

On the HIP path this is five to seven launches per run, each over the whole
run through pointer tables: accumulate/sumsq, select, prepare (decay + the
normalized 16-bit input in both orientations), the Newton-Schulz products,
NorMuon statistics and the fused apply (which also takes a due GPU EMA lerp of
the run's weights). Within ``Dion.step`` the runs queue after the prepare
pass and the step's Newton-Schulz calls run together in grouped launches
(``RunQueue``); the runs are independent, so each run's results are the same.
A user-supplied orthogonalization (``newton_schulz_fn`` replaced) receives the
float32 input rows instead, as the reference's plugin does.
"""

from __future__ import annotations

import math
from collections.abc import Callable
from contextvars import ContextVar
from dataclasses import dataclass
from functools import partial
from typing import Any, Final

import torch
from torch import Tensor

from dionw_amd import _lib, _workspace
from dionw_amd._buckets import Bucket
from dionw_amd._keys import (
    MOMENTUM_FORM_KEY,
    MOMENTUM_KEY,
    MUON_BETA2_KEY,
    ROW_NORMALIZATION_KEY,
    ParamState,
)
from dionw_amd.ema._fusion import ACTIVE_EMA
from dionw_amd.ema.config import ProfileRegion, no_profile
from dionw_amd.matrix_update import MomentumForm, RowNormalization
from dionw_amd.newton_schulz import (
    HipOrthogonalize,
    NewtonSchulzCall,
    group_launches,
    newton_schulz_call,
    padded_sides,
    prepared_inputs,
    prepared_orientations,
    run_newton_schulz,
    run_newton_schulz_call,
    run_newton_schulz_group,
)

__all__ = ["ACTIVE_RUNS", "MAX_RUN_ELEMENTS", "PROFILE_REGION", "RunQueue", "step_run"]

# Named regions of a matrix step (host-side ranges around the launches they
# name, for a profiler's timeline): a run's momentum passes (accumulate, row
# selection, the prepared Newton-Schulz input), the Newton-Schulz products
# (one grouped call or one run's), and a run's finish (NorMuon statistics and
# the weight update).
MOMENTUM_REGION: Final[str] = "dion_momentum"
ORTHOGONALIZE_REGION: Final[str] = "dion_orthogonalize"
FINISH_REGION: Final[str] = "dion_finish"
# Dion.step binds its ``profile_region`` here for the duration of a step.
PROFILE_REGION: ContextVar[ProfileRegion] = ContextVar("dionw_amd_profile_region",
                                                       default=no_profile)

# AdamW update RMS that matrix steps match (Moonshot's 0.2).
ADAMW_UPDATE_RMS: Final[float] = 0.2
# Added to the Frobenius norm before Newton-Schulz.
NEWTON_SCHULZ_EPS: Final[float] = 1e-8
# Largest update (blocks x selected rows x cols) one run orthogonalizes at once.
# The reference caps runs at 2**28 to bound several float32 copies of the update
# on smaller GPUs (_matrix_step.py:40-50). The fused passes here hold no float32
# copy: a run keeps its selected rows in fp16 (in one or both orientations), the
# bf16 output and the Newton-Schulz workspace (six fp16 r x r matrices and one
# r x c per block): at most 20 bytes per update element (square blocks), under
# 22 GB at this cap (17 GB for the Llama-3-8B gate/up bucket). Bigger runs fill
# the 256 CUs better (fewer partly idle tile rounds per product) and launch
# fewer kernels; every Llama-3-8B bucket is one run.
MAX_RUN_ELEMENTS: Final[int] = 2**30


@dataclass
class _Run:
    bucket: Bucket
    params: list[Tensor]        # contiguous parameter storage the kernels write
    writeback: list[tuple[Tensor, Tensor]]  # (parameter, contiguous copy) to copy back
    grads: list[Tensor]         # contiguous float32 gradients
    momentum: Tensor            # [blocks, rows, cols]
    variance: Tensor            # [blocks, rows, 1]

    @property
    def blocks(self) -> int:
        return int(self.momentum.shape[0])


def _make_run(bucket: Bucket, positions: list[int] | range) -> _Run:
    params: list[Tensor] = []
    writeback: list[tuple[Tensor, Tensor]] = []
    grads: list[Tensor] = []
    for i in positions:
        param = bucket.params[i]
        grad = param.grad
        if grad is None:
            raise RuntimeError("every parameter of a Dion run needs a gradient")
        # Channels-last (or otherwise strided) tensors go through row-major copies.
        grads.append(grad.to(torch.float32).contiguous())
        if param.is_contiguous():
            params.append(param.data)
        else:
            copy = param.data.contiguous()
            params.append(copy)
            writeback.append((param.data, copy))
    blocks = bucket.run_blocks(list(positions))
    return _Run(bucket, params, writeback, grads, bucket.momentum[blocks],
                bucket.variance[blocks])


def _step_size(bucket: Bucket, lr: float) -> float:
    """lr times AdamW's update RMS times the Frobenius compensation of a
    partial-row step (_matrix_step.py:147-159)."""
    long_side = max(bucket.rows, bucket.cols)
    short_side = min(bucket.rows, bucket.cols)
    updated_short_side = min(bucket.selected_rows, bucket.cols)
    # The reference's order of evaluation, so that the float32 step is the same.
    return lr * ADAMW_UPDATE_RMS * math.sqrt(long_side) * math.sqrt(short_side / updated_short_side)


# Dion.step sets this around its bucket loop: step_run then queues each fused
# run after its momentum passes, and the queue finishes the queued runs
# together, with one grouped Newton-Schulz call (small runs fill the CUs that
# a large run's products leave idle; each run's results are unchanged).
ACTIVE_RUNS: ContextVar[RunQueue | None] = ContextVar("dionw_amd_active_runs", default=None)

# A queue holds at most this many runs (the library groups up to 8 at a time)
# and this many bytes of Newton-Schulz buffers: queued runs each keep their own.
QUEUE_RUNS: Final[int] = 8
QUEUE_BYTES: Final[int] = 32 * 2**30


def _call_work(call: NewtonSchulzCall) -> float:
    """The F-convention FLOPs of a Newton-Schulz call (a balance weight)."""
    r, c = float(call.r_real), float(call.c_real)
    if call.kind == 0 and c > r:
        return call.blocks * (6.0 * r * r * c + 23.0 * r ** 3)
    return call.blocks * (15.0 * r * r * c + 5.0 * r ** 3)


def _structure(call: NewtonSchulzCall) -> tuple[int, bool, bool]:
    """What decides a call's sequence of products: its kind, the Gram iteration
    (a wide Gram block) or the standard one, and whether the iterate is read as
    it lies (r a multiple of 32)."""
    return call.kind, call.kind == 0 and call.c_real > call.r_real, call.r % 32 == 0


def _lanes(calls: list[NewtonSchulzCall], grouped: bool) -> list[list[int]]:
    """The queued calls split over at most two streams, each list in queue order.

    Grouped, calls of one structure share launches, so each structure stays in
    one lane (the most work on the first); one at a time, the calls are balanced
    by work. One lane when there is nothing to split.
    """
    if len(calls) < 2:
        return [list(range(len(calls)))]
    if grouped:
        classes: dict[tuple[int, bool, bool], list[int]] = {}
        for i, call in enumerate(calls):
            classes.setdefault(_structure(call), []).append(i)
        if len(classes) < 2:
            return [list(range(len(calls)))]
        ordered = sorted(classes.values(), key=lambda ix: -sum(_call_work(calls[i]) for i in ix))
        return [ordered[0], sorted(i for ix in ordered[1:] for i in ix)]
    lanes: list[list[int]] = [[], []]
    load = [0.0, 0.0]
    for i in sorted(range(len(calls)), key=lambda i: -_call_work(calls[i])):
        lane = 0 if load[0] <= load[1] else 1
        lanes[lane].append(i)
        load[lane] += _call_work(calls[i])
    return [sorted(lane) for lane in lanes if lane]


_SIDE_STREAMS: dict[torch.device, torch.cuda.Stream] = {}


def _side_stream(device: torch.device) -> torch.cuda.Stream:
    """A second stream of ``device`` (default priority) for a lane of Newton-Schulz work."""
    side = _SIDE_STREAMS.get(device)
    if side is None:
        side = _SIDE_STREAMS[device] = torch.cuda.Stream(device)
    return side


class RunQueue:
    """Bucket runs waiting for their Newton-Schulz call and the passes after it."""

    def __init__(self) -> None:
        self._calls: list[NewtonSchulzCall] = []
        self._finish: list[Callable[[], None]] = []
        self._bytes = 0
        self._stream: int | None = None
        self._device: torch.device | None = None

    def slot(self, nbytes: int, stream: int, device: torch.device) -> str:
        """Name suffix of the next run's buffers; flushes first if that run does not fit.

        The buffers of queue position ``#i`` are kept from one flush (and step)
        to the next. If growing this position's to ``nbytes`` would take the
        kept total past ``QUEUE_BYTES``, the queue is flushed and every
        position's buffers are dropped first, so the buffers kept never exceed
        ``QUEUE_BYTES`` (or one run's, where a run alone is larger).
        """
        if self._calls and (len(self._calls) >= QUEUE_RUNS or stream != self._stream
                            or self._bytes + nbytes > QUEUE_BYTES):
            self.flush()
        own = f"#{len(self._calls)}"
        kept = _workspace.named_bytes(device, stream, _queued_name)
        mine = _workspace.named_bytes(device, stream,
                                      lambda name: name.partition("#")[2] == own[1:])
        others = kept - mine
        if others > 0 and others + max(mine, nbytes) > QUEUE_BYTES:
            self.flush()
            _workspace.release_named(device, stream, _queued_name)
            own = "#0"
        return own

    def add(self, call: NewtonSchulzCall, finish: Callable[[], None], nbytes: int,
            stream: int, device: torch.device) -> None:
        self._calls.append(call)
        self._finish.append(finish)
        self._bytes += nbytes
        self._stream = stream
        self._device = device

    def flush(self) -> None:
        """Run the queued Newton-Schulz calls and finish the runs.

        The calls go out grouped when that saves launches; then each run's passes
        follow. When grouping saves no launch, each run's iteration is followed
        by its own passes instead, which then find its output still in cache.
        Calls that cannot share launches (different structures, or none grouped)
        run on two streams, the second joining the first at the end: their
        products, each a round of tiles or less on small blocks, then fill the
        CUs together.
        """
        if not self._calls:
            return
        calls, finish, stream, device = self._calls, self._finish, self._stream, self._device
        self._calls, self._finish, self._bytes, self._stream = [], [], 0, None
        grouped = len(calls) > 1 and group_launches(calls) < sum(group_launches([c]) for c in calls)
        lanes = _lanes(calls, grouped)
        if len(lanes) == 1:
            _run_lane(calls, finish, lanes[0], grouped, stream)
            return
        main = torch.cuda.current_stream(device)
        side = _side_stream(device)
        side.wait_stream(main)
        for lane, lane_stream in zip(lanes, (main, side)):
            with torch.cuda.stream(lane_stream):
                _run_lane(calls, finish, lane, grouped, lane_stream.cuda_stream)
        main.wait_stream(side)


def _run_lane(calls: list[NewtonSchulzCall], finish: list[Callable[[], None]], lane: list[int],
              grouped: bool, stream: int) -> None:
    """The calls ``lane`` of the queue, then (or each followed by) their runs' passes."""
    region = PROFILE_REGION.get()
    mine = [calls[i] for i in lane]
    if grouped and len(mine) > 1 and group_launches(mine) < sum(group_launches([c]) for c in mine):
        with region(ORTHOGONALIZE_REGION):
            run_newton_schulz_group(mine, stream)
        for i in lane:
            finish[i]()
        return
    for i in lane:
        with region(ORTHOGONALIZE_REGION):
            run_newton_schulz_call(calls[i], stream)
        finish[i]()


def _queued_name(name: str) -> bool:
    """Whether a scratch buffer belongs to a queue position (``#i`` suffix)."""
    return "#" in name


def _ns_bytes(ortho: HipOrthogonalize, blocks: int, k: int, cols: int) -> int:
    """Bytes of a fused run's Newton-Schulz buffers (inputs, output, workspace)."""
    p_pad, j_pad = padded_sides(k, cols)
    r, c = min(p_pad, j_pad), max(p_pad, j_pad)
    work = int(_lib.library().dionw_newton_schulz_workspace(ortho.lib_kind, blocks, r, c))
    inputs = sum(prepared_orientations(k, cols))
    return inputs * 2 * blocks * p_pad * j_pad + 2 * blocks * k * cols + work


def step_run(
    bucket: Bucket, positions: list[int] | range, group: dict[str, Any], state: ParamState
) -> None:
    """Apply one Dion step to the consecutive bucket parameters ``positions``.

    Inside ``Dion.step`` a fused run is queued after its momentum passes and
    finished when the step's queue is flushed.

    Raises:
        RuntimeError: If a parameter of the run lacks a gradient.
    """
    del state  # the run's momentum and variance are views of the bucket
    run = _make_run(bucket, positions)
    lr = float(group["lr"])
    step = -_step_size(bucket, lr)
    device = run.momentum.device
    stream = _lib.stream_handle(device)
    blocks, rows, cols, k = run.blocks, bucket.rows, bucket.cols, bucket.selected_rows
    count = len(run.grads)
    per_param = bucket.blocks_per_param
    mu = float(group[MOMENTUM_KEY])
    nesterov = MomentumForm(group[MOMENTUM_FORM_KEY]) is MomentumForm.NESTEROV
    ortho = bucket.orthogonalize
    fused = isinstance(ortho, HipOrthogonalize)
    safety = ortho.norm_safety if fused else 1.0
    # The element type of the iteration fixes how its input norm rounds.
    norm_elem = ortho.elem if fused else _lib.F32
    grads = _lib.ptr_array(run.grads)
    momentum = run.momentum
    queue = ACTIVE_RUNS.get() if fused else None
    nbytes = _ns_bytes(ortho, blocks, k, cols) if queue is not None else 0
    # Buffers still in use when a queued run finishes get names of their own.
    own = queue.slot(nbytes, stream, device) if queue is not None else ""

    region = PROFILE_REGION.get()
    with region(MOMENTUM_REGION):
        den = _workspace.buffer(device, "den", (blocks,), torch.float32)
        rowsq = _workspace.buffer(device, "rowsq", (blocks * rows,), torch.float32)
        selected = k < rows
        idx = slot = None
        if selected:
            scores = _workspace.buffer(device, "scores", (blocks * rows,), torch.float32)
            idx = _workspace.buffer(device, "idx" + own, (blocks, k), torch.int32)
            slot = _workspace.buffer(device, "slot" + own, (blocks, rows), torch.int32)
            _lib.call("dionw_accumulate_scores", grads, count, per_param * rows, cols,
                      momentum.data_ptr(), scores.data_ptr(), rowsq.data_ptr(), norm_elem, stream)
            _lib.call("dionw_select_rows", scores.data_ptr(), rowsq.data_ptr(), blocks, rows, k,
                      safety, NEWTON_SCHULZ_EPS, idx.data_ptr(), slot.data_ptr(), den.data_ptr(),
                      norm_elem, stream)
        elif fused:
            _lib.call("dionw_full_sumsq", grads, count, per_param * rows, cols,
                      momentum.data_ptr(), mu, int(nesterov), rowsq.data_ptr(), norm_elem, stream)
            _lib.call("dionw_block_denom", rowsq.data_ptr(), blocks, rows, safety,
                      NEWTON_SCHULZ_EPS, den.data_ptr(), norm_elem, stream)
        idx_ptr = None if idx is None else idx.data_ptr()
        if fused:
            # Only the orientations the iteration reads are written.
            xr, xt = prepared_inputs(ortho, device, blocks, k, cols, "ns_xr" + own,
                                     "ns_xt" + own)
            _lib.call("dionw_prepare_ns_input", grads, count, momentum.data_ptr(), idx_ptr,
                      den.data_ptr(), blocks, rows, cols, k, *padded_sides(k, cols), mu,
                      int(nesterov), 1, ortho.elem, None if xr is None else xr.data_ptr(),
                      None if xt is None else xt.data_ptr(), stream)
        else:
            raw = torch.empty(blocks, k, cols, device=device, dtype=torch.float32)
            _lib.call("dionw_prepare_ns_input", grads, count, momentum.data_ptr(), idx_ptr,
                      den.data_ptr(), blocks, rows, cols, k, k, cols, mu, int(nesterov), 1,
                      _lib.F32, raw.data_ptr(), None, stream)

    if fused:
        orthogonal = _workspace.buffer(device, "ns_out" + own, (blocks, k, cols), torch.bfloat16)
        if queue is not None:
            call = newton_schulz_call(ortho, blocks, k, cols, xr, xt, orthogonal,
                                      "ns_workspace" + own)
            queue.add(call, partial(_finish_run, run, bucket, positions, group, orthogonal, idx,
                                    slot, step), nbytes, stream, device)
            return
        with region(ORTHOGONALIZE_REGION):
            run_newton_schulz(ortho, blocks, k, cols, xr, xt, orthogonal, stream)
    else:
        with region(ORTHOGONALIZE_REGION):
            orthogonal = ortho(raw, NEWTON_SCHULZ_EPS)
            orthogonal = orthogonal.to(torch.bfloat16).contiguous()
    _finish_run(run, bucket, positions, group, orthogonal, idx, slot, step)


def _finish_run(
    run: _Run,
    bucket: Bucket,
    positions: list[int] | range,
    group: dict[str, Any],
    orthogonal: Tensor,
    idx: Tensor | None,
    slot: Tensor | None,
    step: float,
) -> None:
    """NorMuon statistics and the weight update of a run whose orthogonalized
    rows ``orthogonal`` ([blocks, k, cols] bf16) are ready (_matrix_step.py:274-311),
    on torch's current stream (the queue may finish a run on its second stream)."""
    with PROFILE_REGION.get()(FINISH_REGION):
        device = run.momentum.device
        stream = _lib.stream_handle(device)
        blocks, rows, cols, k = run.blocks, bucket.rows, bucket.cols, bucket.selected_rows
        count = len(run.params)
        per_param = bucket.blocks_per_param
        lr = float(group["lr"])
        idx_ptr = None if idx is None else idx.data_ptr()
        rowd = scale = None
        match RowNormalization(group[ROW_NORMALIZATION_KEY]):
            case RowNormalization.NORMUON:
                rowd = _workspace.buffer(device, "rowd", (blocks, k), torch.float32)
                scratch = _workspace.buffer(device, "row_scratch", (2 * blocks * k,), torch.float32)
                scale = _workspace.buffer(device, "scale", (blocks,), torch.float32)
                _lib.call("dionw_normuon_stats", orthogonal.data_ptr(), blocks, k, rows, cols,
                          idx_ptr, run.variance.data_ptr(), float(group[MUON_BETA2_KEY]), step,
                          rowd.data_ptr(), scratch.data_ptr(), scale.data_ptr(), stream)
            case RowNormalization.NONE:
                pass
            case _ as unreachable:
                raise RuntimeError(f"no row normalization named {unreachable}")

        weight_decay = float(group["weight_decay"])
        decay = 1.0 - lr * weight_decay
        common = (count, per_param, rows, cols, k, orthogonal.data_ptr(), idx_ptr,
                  _lib.ptr(slot), _lib.ptr(rowd), _lib.ptr(scale), step, decay,
                  int(weight_decay > 0.0))
        # A due GPU EMA lerp of these weights rides on the apply pass (one pass
        # instead of apply then EMA; the same lerp arithmetic).
        ema = ACTIVE_EMA.get()
        params = [bucket.params[i] for i in positions]
        fusable = ema is not None and not run.writeback
        shadows = ema.fusable_shadows(params) if fusable else None
        # A due CPU EMA's host snapshots may be written by the same pass (the new
        # weights go to HBM and over the host link at once) instead of copied after it.
        staged = ema.stageable_buffers(params) if fusable and ema.fuse_host_copies else None
        if shadows is not None:
            _lib.call("dionw_apply_update_ema", _lib.ptr_array(run.params), _lib.ptr_array(shadows),
                      *common, ema.fused_weight(), stream)
            ema.mark_fused(params)
        elif staged is not None:
            _lib.call("dionw_apply_update_stage", _lib.ptr_array(run.params),
                      _lib.ptr_array(staged), *common, stream)
            ema.mark_staged(params)
        else:
            _lib.call("dionw_apply_update", _lib.ptr_array(run.params), *common, stream)
        for param, copy in run.writeback:
            param.copy_(copy)
        if ema is not None:
            ema.stage_written(params)
