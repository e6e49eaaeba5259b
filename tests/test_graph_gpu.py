"""One ``Dion.step`` recorded as a HIP graph and replayed (GPU).

Two optimizers start from the same parameters and gradients: one steps
eagerly, the other replays its recorded step. Between steps the test does its
own eager work (new gradients written into the recorded ``.grad`` tensors,
synchronizations), and every replay must equal the eager step bit for bit:
parameters, Dion momentum and variance, AdamW moments and step counters.
The model mixes what a step can issue: a selected-rows Gram run, an every-row
run whose square blocks take the standard iteration on a second stream, a
Polar Express group and AdamW parameters.
"""

from __future__ import annotations

import pytest
import torch
from torch import nn

from dionw_amd import EMAConfig, FRACTION_KEY, NEWTON_SCHULZ_KEY, ROUTE_KEY, Dion, StepGraph

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _model(seed: int) -> tuple[list[dict], list[nn.Parameter]]:
    g = torch.Generator(device=DEV).manual_seed(seed)

    def param(*shape: int) -> nn.Parameter:
        p = nn.Parameter(torch.empty(*shape, device=DEV).normal_(0.0, 0.02, generator=g))
        p.grad = torch.zeros_like(p)
        return p

    selected = [param(1024, 512) for _ in range(3)]        # k = 256 of 1024 rows, Gram
    wide = [param(384, 1536) for _ in range(2)]            # every row, wide Gram
    square = [param(384, 384) for _ in range(2)]           # every row, standard iteration
    quintic = [param(256, 768) for _ in range(2)]          # Polar Express
    vectors = [param(512), param(384), param(1000, 64)]
    groups = [
        {"params": selected, ROUTE_KEY: "matrix", FRACTION_KEY: 0.25},
        {"params": wide + square, ROUTE_KEY: "matrix", FRACTION_KEY: 1.0},
        {"params": quintic, ROUTE_KEY: "matrix", FRACTION_KEY: 1.0,
         NEWTON_SCHULZ_KEY: "polar_express"},
        {"params": vectors, ROUTE_KEY: "adamw"},
    ]
    return groups, selected + wide + square + quintic + vectors


def _dion(groups: list[dict], **kwargs) -> Dion:
    return Dion(groups, lr=2e-3, weight_decay=0.05, momentum=0.95, muon_beta2=0.95,
                betas=(0.9, 0.95), eps=1e-8, **kwargs)


def _same(name: str, a: Dion, b: Dion, pa: list[nn.Parameter], pb: list[nn.Parameter]) -> None:
    for i, (x, y) in enumerate(zip(pa, pb)):
        assert torch.equal(x.detach(), y.detach()), f"{name}: parameter {i}"
        sa, sb = a.state[x], b.state[y]
        assert sa.keys() == sb.keys(), f"{name}: state keys of parameter {i}"
        for key in sa:
            assert torch.equal(sa[key], sb[key]), f"{name}: {key} of parameter {i}"


def test_replays_equal_eager_steps_bit_for_bit() -> None:
    groups_a, params_a = _model(0)
    groups_b, params_b = _model(0)
    eager, recorded = _dion(groups_a), _dion(groups_b)
    g = torch.Generator(device=DEV).manual_seed(1)
    grads = [torch.empty_like(p).normal_(0.0, 1e-3, generator=g) for p in params_a]
    for pa, pb, gr in zip(params_a, params_b, grads):
        pa.grad.copy_(gr)
        pb.grad.copy_(gr)
    # One eager step each: packs the state and sizes the scratch.
    eager.step()
    recorded.step()
    torch.cuda.synchronize()
    graph = StepGraph(recorded)
    torch.cuda.synchronize()
    _same("after recording (nothing ran)", eager, recorded, params_a, params_b)
    for step in range(6):
        for pa, pb in zip(params_a, params_b):
            new = torch.empty_like(pa).normal_(0.0, 1e-3, generator=g)
            pa.grad.copy_(new)
            pb.grad.copy_(new)
        eager.step()
        graph.replay()
        torch.cuda.synchronize()
        _same(f"step {step}", eager, recorded, params_a, params_b)


def test_a_step_that_would_pack_or_run_an_ema_is_not_recorded() -> None:
    groups, params = _model(2)
    fresh = _dion(groups)
    for p in params:
        p.grad.normal_(0.0, 1e-3)
    graph = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="not packed"):
        with torch.cuda.graph(graph):
            fresh.step()
    torch.cuda.synchronize()
    groups, params = _model(3)
    with_ema = _dion(groups, ema=EMAConfig(decay=0.99))
    for p in params:
        p.grad.normal_(0.0, 1e-3)
    with_ema.step()
    with pytest.raises(RuntimeError, match="EMA"):
        StepGraph(with_ema)
