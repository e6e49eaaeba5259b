"""Grouped Newton-Schulz launches against separate calls (GPU).

``Dion.step`` queues its bucket runs and orthogonalizes them with one
``dionw_newton_schulz_group`` call: the same products of several runs share a
launch. Every tile computes the same sums in the same order either way, so the
results must be bit-identical to one ``dionw_newton_schulz`` call per run, and
a step with the queue must equal a step without it. Edge cases: tall and
ragged blocks, depths that are not multiples of 64 (those products fall back
to one launch per run), square blocks and the bf16 quintics (other product
sequences, grouped separately), and more runs than one group holds.
"""

from __future__ import annotations

import contextvars

import pytest
import torch
from torch import nn

import dionw_amd._matrix_step
import dionw_amd.optimizer
from dionw_amd import (
    FRACTION_KEY,
    ROUTE_KEY,
    Dion,
    EMAConfig,
    MatrixUpdate,
    MomentumForm,
    NewtonSchulz,
    RouteKind,
    RowNormalization,
    _lib,
)
from dionw_amd.newton_schulz import (
    newton_schulz_call,
    newton_schulz_fn,
    prepared_orientations,
    run_newton_schulz,
    run_newton_schulz_group,
)

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _round8(n: int) -> int:
    return (n + 7) // 8 * 8


def _inputs(kind: NewtonSchulz, blocks: int, rows: int, cols: int, seed: int):
    """Normalized iteration inputs in both orientations, zero padding."""
    ortho = newton_schulz_fn(kind)
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(blocks, rows, cols, generator=g)
    x = x / (x.flatten(1).norm(dim=1).view(-1, 1, 1) + 1e-8)
    xr = torch.zeros(blocks, _round8(rows), _round8(cols))
    xr[:, :rows, :cols] = x
    xr = xr.to(ortho.dtype)
    return ortho, xr, xr.mT.contiguous()


RUNS = [  # (kind, blocks, rows, cols)
    (NewtonSchulz.GRAM, 3, 256, 1024),
    (NewtonSchulz.GRAM, 2, 512, 768),
    (NewtonSchulz.GRAM, 4, 64, 512),
    (NewtonSchulz.GRAM, 2, 1024, 256),   # tall: iterates on the transpose
    (NewtonSchulz.GRAM, 2, 100, 200),    # ragged, depth 104: one launch per run
    (NewtonSchulz.GRAM, 2, 256, 256),    # square: the standard iteration
    (NewtonSchulz.POLAR_EXPRESS, 2, 128, 512),
    (NewtonSchulz.KELLER, 3, 256, 768),
]


@pytest.mark.parametrize("runs", [RUNS, RUNS[:3], RUNS[:1]], ids=["mixed", "gram", "one"])
def test_group_call_equals_separate_calls(runs) -> None:
    stream = _lib.stream_handle(torch.device(DEV))
    separate, grouped, calls, inputs = [], [], [], []
    for i, (kind, blocks, rows, cols) in enumerate(runs):
        ortho, xr, xt = _inputs(kind, blocks, rows, cols, seed=i)
        out = torch.empty(blocks, rows, cols, dtype=torch.bfloat16, device=DEV)
        print(f"run {i}: {kind.value} {blocks}x{rows}x{cols}", flush=True)
        run_newton_schulz(ortho, blocks, rows, cols, xr.to(DEV), xt.to(DEV), out, stream)
        separate.append(out)
        out2 = torch.empty_like(out)
        # A call holds addresses only: its buffers must outlive the grouped launch.
        # The grouped leg passes only the inputs the iteration reads, the separate
        # leg both (an unread transpose is ignored).
        want_xr, want_xt = prepared_orientations(rows, cols)
        xr_d = xr.to(DEV) if want_xr else None
        xt_d = xt.to(DEV) if want_xt else None
        inputs.append((xr_d, xt_d))
        calls.append(newton_schulz_call(ortho, blocks, rows, cols, xr_d, xt_d, out2,
                                        f"test_group_ws#{i}"))
        grouped.append(out2)
    run_newton_schulz_group(calls, stream)
    torch.cuda.synchronize()
    for (kind, blocks, rows, cols), a, b in zip(runs, separate, grouped):
        assert torch.isfinite(a.float()).all()
        assert torch.equal(a.cpu(), b.cpu()), f"{kind.value} {blocks}x{rows}x{cols} differs"


class _Net(nn.Module):
    """Buckets of wide, tall, ragged and square blocks."""

    def __init__(self) -> None:
        super().__init__()
        self.a = nn.Linear(1024, 256, bias=False)
        self.b = nn.Linear(1024, 256, bias=False)
        self.c = nn.Linear(256, 1024, bias=False)
        self.d = nn.Linear(700, 300, bias=False)
        self.e = nn.Linear(512, 512, bias=False)
        self.f = nn.Linear(2048, 384, bias=False)


def _step_twice(kind: NewtonSchulz, fraction: float, queued: bool, ema: bool,
                monkeypatch) -> tuple[list[torch.Tensor], list[torch.Tensor]]:
    torch.manual_seed(0)
    net = _Net().to(DEV)
    opt = Dion(
        [{"params": list(net.parameters()), ROUTE_KEY: RouteKind.MATRIX.value,
          FRACTION_KEY: fraction}],
        lr=1e-3, momentum=0.95, muon_beta2=0.95, weight_decay=0.1,
        matrix_update=MatrixUpdate(kind, RowNormalization.NORMUON, MomentumForm.HEAVY_BALL),
        ema=EMAConfig(decay=0.99) if ema else None,
    )
    with monkeypatch.context() as m:
        if not queued:
            # step_run reads a variable the optimizer never sets: no queue.
            m.setattr(dionw_amd._matrix_step, "ACTIVE_RUNS",
                      contextvars.ContextVar("unset", default=None))
        g = torch.Generator(device=DEV).manual_seed(1)
        for _ in range(2):
            for p in net.parameters():
                p.grad = torch.randn(p.shape, device=DEV, generator=g) * 1e-3
            opt.step()
    torch.cuda.synchronize()
    params = [p.detach().cpu().clone() for p in net.parameters()]
    state = [opt.state[p]["momentum"].cpu().clone() for p in net.parameters()]
    return params, state


@pytest.mark.parametrize(("kind", "fraction", "ema"), [
    (NewtonSchulz.GRAM, 0.25, False),
    (NewtonSchulz.GRAM, 1.0, True),
    (NewtonSchulz.POLAR_EXPRESS, 0.5, False),
])
def test_queued_step_equals_unqueued_step(kind, fraction, ema, monkeypatch) -> None:
    a_params, a_state = _step_twice(kind, fraction, True, ema, monkeypatch)
    b_params, b_state = _step_twice(kind, fraction, False, ema, monkeypatch)
    for x, y in zip(a_params, b_params):
        assert torch.equal(x, y), "parameters differ"
    for x, y in zip(a_state, b_state):
        assert torch.equal(x, y), "momentum differs"


def test_queue_flushes_when_full(monkeypatch) -> None:
    """One bucket split into single-parameter runs: more runs than a group holds."""
    monkeypatch.setattr(dionw_amd.optimizer, "MAX_RUN_ELEMENTS", 1)
    torch.manual_seed(0)
    params = [nn.Parameter(torch.randn(256, 512, device=DEV) * 0.02) for _ in range(11)]
    copies = [nn.Parameter(p.detach().clone()) for p in params]

    def make(ps):
        return Dion([{"params": ps, ROUTE_KEY: RouteKind.MATRIX.value, FRACTION_KEY: 0.25}],
                    lr=1e-3, weight_decay=0.1)

    opt, ref = make(params), make(copies)
    g = torch.Generator(device=DEV).manual_seed(2)
    grads = [torch.randn(256, 512, device=DEV, generator=g) * 1e-3 for _ in params]
    for p, c, gr in zip(params, copies, grads):
        p.grad, c.grad = gr.clone(), gr.clone()
    opt.step()
    with monkeypatch.context() as m:
        m.setattr(dionw_amd._matrix_step, "ACTIVE_RUNS",
                  contextvars.ContextVar("unset", default=None))
        ref.step()
    torch.cuda.synchronize()
    for p, c in zip(params, copies):
        assert torch.equal(p.detach().cpu(), c.detach().cpu())
