"""``Dion.step`` on the HIP path against the CPU oracle and the reference's invariants (GPU).

Restates the reference's optimizer tests (tests/test_optimizer.py) without
microsoft/dion: the Newton-Schulz plugin is replaced by the exact polar factor
(as test_optimizer.py:90-132 does) to pin every other stage to float32
rounding, and the HIP Newton-Schulz is checked against the oracle's.
"""

from __future__ import annotations

import io
import math

import numpy as np
import pytest
import torch
from torch import nn

import dionw_amd
import dionw_amd._buckets
from dionw_amd import (
    FRACTION_KEY,
    NUM_HEADS_KEY,
    ROUTE_KEY,
    Dion,
    EMAConfig,
    MatrixUpdate,
    MomentumForm,
    NewtonSchulz,
    RouteKind,
    RowNormalization,
)
from oracle import dion_ref
from tests.conftest import rel_fro

pytestmark = pytest.mark.gpu
DEV = "cuda"
LR = 1e-3


def _exact_polar_bf16(x: torch.Tensor, epsilon: float) -> torch.Tensor:
    del epsilon
    return dion_ref.exact_polar(x.cpu()).to(device=x.device, dtype=torch.bfloat16)


def _dion(params, fraction, *, kind=NewtonSchulz.GRAM, weight_decay=0.0, normuon=True,
          nesterov=False, heads=None, ema=None) -> Dion:
    return Dion(
        [{"params": list(params), ROUTE_KEY: RouteKind.MATRIX.value, FRACTION_KEY: fraction,
          NUM_HEADS_KEY: heads}],
        lr=LR, momentum=0.95, muon_beta2=0.95, betas=(0.9, 0.99), weight_decay=weight_decay,
        eps=1e-8,
        matrix_update=MatrixUpdate(
            kind,
            RowNormalization.NORMUON if normuon else RowNormalization.NONE,
            MomentumForm.NESTEROV if nesterov else MomentumForm.HEAVY_BALL,
        ),
        ema=ema,
    )


CASES = [((256, 512), 0.25), ((64, 128), 1.0), ((64, 128), 0.5), ((256, 64), 0.5),
         ((128, 128), 0.25), ((160, 96), 1.0),
         # sides that are not multiples of 8 or 4 (padded Newton-Schulz input,
         # scalar row loads), and a long block (16384 rows, top-4096 selection)
         ((100, 70), 0.3), ((37, 61), 1.0), ((16384, 128), 0.25),
         # a single selected row (k = 1), and a single-row block
         ((64, 128), 1.0 / 64), ((1, 96), 1.0)]


@pytest.mark.parametrize("weight_decay", [0.0, 0.1])
@pytest.mark.parametrize(("shape", "fraction"), CASES)
def test_exact_polar_step_matches_oracle(shape, fraction, weight_decay, monkeypatch) -> None:
    """With Newton-Schulz replaced by the exact polar factor, the GPU step and
    the oracle agree to float32 rounding over 4 steps (two same-shape params)."""
    monkeypatch.setattr(dionw_amd._buckets, "newton_schulz_fn", lambda _kind: _exact_polar_bf16)
    g = torch.Generator().manual_seed(0)
    starts = [torch.randn(*shape, generator=g) * 0.02 for _ in range(2)]
    params = [nn.Parameter(s.clone().to(DEV)) for s in starts]
    opt = _dion(params, fraction, weight_decay=weight_decay)
    rows, cols = shape
    k = min(rows, math.ceil(fraction * rows))
    w = torch.stack(starts)
    mom = torch.zeros_like(w)
    var = torch.zeros(2, rows, 1)
    for step in range(4):
        grads = torch.randn(2, *shape, generator=g)
        for p, gr in zip(params, grads):
            p.grad = gr.to(DEV)
        opt.step()
        dion_ref.step_blocks(w, grads, mom, var, k=k, lr=LR, mu=0.95, beta2=0.95,
                             weight_decay=weight_decay, orthogonalize=_exact_polar_cpu)
        got_m = torch.stack([opt.state[p]["momentum"].cpu() for p in params])
        assert torch.equal(got_m, mom), f"step {step}: momentum differs (selection?)"
        got_w = torch.stack([p.detach().cpu() for p in params])
        torch.testing.assert_close(got_w, w, rtol=0, atol=2e-7, msg=f"step {step}: weights")


def _exact_polar_cpu(x: torch.Tensor, epsilon: float) -> torch.Tensor:
    del epsilon
    return dion_ref.exact_polar(x).to(torch.bfloat16)


@pytest.mark.parametrize("kind", [NewtonSchulz.GRAM, NewtonSchulz.POLAR_EXPRESS, NewtonSchulz.KELLER_TRITON])
@pytest.mark.parametrize(("shape", "fraction", "heads"), [
    ((1024, 1024), 1.0, None), ((512, 1024), 0.25, None), ((768, 256), 1.0, 3),
    ((1408, 512), 0.25, None),
    # 30 x 70 selected blocks (padded to 32 x 72): at this size the oracle's own
    # fp16 Gram iteration is ~1e-2 from the float64 polynomial.
    ((100, 70), 0.3, None),
    # Short sides that are odd multiples of 32 next to a long side less than 32
    # longer (no padding to 64-deep stages): square, near-square (where Gram's
    # rounding error is ~1.6e-2), tall, and a selected k = 288 beside 296 columns.
    ((288, 288), 1.0, None), ((288, 296), 1.0, None), ((296, 288), 1.0, None),
    ((1152, 296), 0.25, None),
    # one selected row: a 1 x 128 iterate (padded to 8 rows)
    ((64, 128), 1.0 / 64, None)])
def test_hip_step_matches_oracle(kind, shape, fraction, heads) -> None:
    """The full HIP step (Newton-Schulz included) against the oracle: selection
    and momentum bit-exact, parameters within the north-star 2e-3, and the
    update within a bar derived from the oracle's own Newton-Schulz rounding at
    that step: ``1.6 e + 3e-3``, where ``e`` is the oracle output's distance to
    the same polynomials in float64 on the same input (two roundings at the
    same points, in another accumulation order). ``e`` is 0.002-0.004 for
    Gram, ~0.015 for the bf16 Keller quintic and ~0.03 for POLAR_EXPRESS, which
    rounds its products to bf16 before the elementwise terms (the reference's
    cuBLAS quintic)."""
    from tests.test_kernels_gpu import POLYNOMIALS

    seen = {}

    def recording_oracle(x: torch.Tensor, epsilon: float) -> torch.Tensor:
        out = dion_ref.ORTHOGONALIZE[kind.value](x, epsilon)
        tall = x.shape[-2] > x.shape[-1]
        target = dion_ref.polynomial_float64(x.mT if tall else x, *POLYNOMIALS[kind])
        seen["rounding"] = rel_fro(out.float(), target.mT if tall else target)
        return out

    g = torch.Generator().manual_seed(1)
    start = torch.randn(*shape, generator=g) * 0.02
    param = nn.Parameter(start.clone().to(DEV))
    opt = _dion([param], fraction, kind=kind, weight_decay=0.05, heads=heads)
    blocks = heads or 1
    rows, cols = shape[0] // blocks, shape[1]
    k = min(rows, math.ceil(fraction * rows))
    w = start.view(blocks, rows, cols).clone()
    mom = torch.zeros_like(w)
    var = torch.zeros(blocks, rows, 1)
    for step in range(3):
        grad = torch.randn(*shape, generator=g) * 1e-3
        param.grad = grad.to(DEV)
        before = param.detach().cpu().view(blocks, rows, cols).clone()
        opt.step()
        w_ref_before = w.clone()
        dion_ref.step_blocks(w, grad.view(blocks, rows, cols), mom, var, k=k, lr=LR, mu=0.95,
                             beta2=0.95, weight_decay=0.05, kind=kind.value,
                             orthogonalize=recording_oracle)
        got_m = opt.state[param]["momentum"].cpu().view(blocks, rows, cols)
        assert torch.equal(got_m, mom), f"step {step}: momentum (selection) differs"
        decay = 1.0 - LR * 0.05
        upd_gpu = param.detach().cpu().view(blocks, rows, cols) - before * decay
        upd_ref = w - w_ref_before * decay
        err = rel_fro(upd_gpu, upd_ref)
        bar = 1.6 * seen["rounding"] + 3e-3
        assert err < bar, (f"step {step} {kind.value} {shape}: update rel err {err}, bar {bar} "
                           f"(oracle rounding {seen['rounding']})")
        assert rel_fro(param.detach().cpu().view(blocks, rows, cols), w) < 2e-3
        got_v = opt.state[param]["variance"].cpu().view(blocks, rows, 1)
        assert rel_fro(got_v, var) < 2e-2, f"step {step}: variance"
        w = param.detach().cpu().view(blocks, rows, cols).clone()  # follow the GPU trajectory


def test_lr_zero_freezes_weights() -> None:
    g = torch.Generator().manual_seed(2)
    param = nn.Parameter((torch.randn(128, 256, generator=g) * 0.02).to(DEV))
    start = param.detach().clone()
    opt = Dion([{"params": [param], ROUTE_KEY: "matrix", FRACTION_KEY: 0.5}], lr=0.0,
               weight_decay=0.1)
    for _ in range(2):
        param.grad = torch.randn(128, 256, generator=g).to(DEV)
        opt.step()
    assert torch.equal(param.detach(), start)


def test_weight_decay_exact_on_zero_gradients() -> None:
    param = nn.Parameter(torch.randn(64, 128).to(DEV) * 0.02)
    start = param.detach().clone()
    opt = Dion([{"params": [param], ROUTE_KEY: "matrix", FRACTION_KEY: 0.5}], lr=1e-2,
               weight_decay=0.1)
    param.grad = torch.zeros_like(param)
    opt.step()
    assert torch.equal(param.detach(), start * (1.0 - 1e-2 * 0.1))


def test_same_shape_momenta_share_storage() -> None:
    params = [nn.Parameter(torch.randn(32, 32, device=DEV)) for _ in range(2)]
    opt = _dion(params, 1.0)
    for p in params:
        p.grad = torch.randn_like(p)
    opt.step()
    storages = {opt.state[p]["momentum"].untyped_storage().data_ptr() for p in params}
    assert len(storages) == 1
    assert opt.state[params[0]]["momentum"].untyped_storage().nbytes() == 2 * 32 * 32 * 4


def test_release_workspace_by_index_less_device_frees_the_step_scratch() -> None:
    """``release_workspace('cuda')`` frees the scratch a step left on the current
    GPU (kept under ``cuda:<index>``), and a later step regrows it."""
    from dionw_amd import _workspace

    param = nn.Parameter(torch.randn(256, 512, device=DEV) * 0.02)
    opt = _dion([param], 0.25)
    param.grad = torch.randn_like(param)
    opt.step()
    torch.cuda.synchronize()
    assert _workspace.held_bytes("cuda") > 0
    here = f"cuda:{torch.cuda.current_device()}"
    assert _workspace.held_bytes("cuda") == _workspace.held_bytes(here)
    dionw_amd.release_workspace("cuda")
    assert _workspace.held_bytes("cuda") == 0
    opt.step()
    torch.cuda.synchronize()
    assert _workspace.held_bytes("cuda") > 0


def test_resume_is_bit_exact() -> None:
    def model():
        torch.manual_seed(3)
        return nn.Sequential(nn.Linear(256, 512), nn.GELU(), nn.Linear(512, 128)).to(DEV)

    def run(steps, opt, m, g):
        for _ in range(steps):
            for p in m.parameters():
                p.grad = torch.randn(p.shape, generator=g).to(DEV) * 1e-3
            opt.step()

    m1 = model()
    groups, _ = dionw_amd.param_groups(m1, fraction=0.5, selection_min_dim=128)
    o1 = Dion(groups, lr=1e-3, weight_decay=0.05, ema=EMAConfig(decay=0.9))
    run(4, o1, m1, torch.Generator().manual_seed(9))

    m2 = model()
    groups, _ = dionw_amd.param_groups(m2, fraction=0.5, selection_min_dim=128)
    o2 = Dion(groups, lr=1e-3, weight_decay=0.05, ema=EMAConfig(decay=0.9))
    gen = torch.Generator().manual_seed(9)
    run(2, o2, m2, gen)
    buf = io.BytesIO()
    torch.save({"model": m2.state_dict(), "opt": o2.state_dict()}, buf)
    buf.seek(0)
    saved = torch.load(buf, weights_only=True)
    m3 = model()
    m3.load_state_dict(saved["model"])
    groups, _ = dionw_amd.param_groups(m3, fraction=0.5, selection_min_dim=128)
    o3 = Dion(groups, lr=1e-3, weight_decay=0.05, ema=EMAConfig(decay=0.9))
    o3.load_state_dict(saved["opt"])
    run(2, o3, m3, gen)
    for a, b in zip(m1.parameters(), m3.parameters()):
        assert torch.equal(a, b)
    for a, b in zip(m1.parameters(), m3.parameters()):
        assert torch.equal(o1.state[a]["ema_shadow"], o3.state[b]["ema_shadow"])


def test_adamw_route_matches_torch_fused_adamw() -> None:
    torch.manual_seed(4)
    vec = nn.Parameter(torch.randn(300, device=DEV))
    ref = nn.Parameter(vec.detach().clone())
    opt = Dion([{"params": [vec], ROUTE_KEY: "adamw"}], lr=1e-3, betas=(0.9, 0.99),
               weight_decay=0.1, eps=1e-8)
    torch_opt = torch.optim.AdamW([ref], lr=1e-3, betas=(0.9, 0.99), weight_decay=0.1, eps=1e-8,
                                  fused=True)
    for _ in range(5):
        grad = torch.randn(300, device=DEV)
        vec.grad, ref.grad = grad.clone(), grad.clone()
        opt.step()
        torch_opt.step()
        assert torch.equal(vec, ref)


def test_runs_split_by_missing_gradients_match_lone_params() -> None:
    g = torch.Generator().manual_seed(5)
    starts = [torch.randn(64, 96, generator=g) * 0.02 for _ in range(3)]
    grads = [torch.randn(64, 96, generator=g) for _ in range(3)]
    together = [nn.Parameter(s.clone().to(DEV)) for s in starts]
    opt = _dion(together, 0.5)
    together[0].grad, together[2].grad = grads[0].to(DEV), grads[2].to(DEV)
    opt.step()
    for i in (0, 2):
        lone = nn.Parameter(starts[i].clone().to(DEV))
        lone_opt = _dion([lone], 0.5)
        lone.grad = grads[i].to(DEV)
        lone_opt.step()
        assert torch.equal(lone.detach(), together[i].detach()), f"param {i}"
    assert torch.equal(together[1].detach().cpu(), starts[1])


def test_runs_above_the_element_cap_step_like_lone_parameters(monkeypatch) -> None:
    """A bucket above ``MAX_RUN_ELEMENTS`` steps in runs below the cap, and each
    parameter gets the step it would get alone (tests/test_optimizer.py:687-728;
    the exact polar factor pins every other stage to float32 rounding)."""
    import dionw_amd.optimizer as optimizer_module

    monkeypatch.setattr(dionw_amd._buckets, "newton_schulz_fn", lambda _kind: _exact_polar_bf16)
    monkeypatch.setattr(optimizer_module, "MAX_RUN_ELEMENTS", 2 * 32 * 48)  # two blocks per run
    runs: list[int] = []
    real_step_run = optimizer_module.step_run

    def counted(bucket, positions, group, state):
        runs.append(len(positions))
        real_step_run(bucket, positions, group, state)

    monkeypatch.setattr(optimizer_module, "step_run", counted)
    g = torch.Generator().manual_seed(9)
    starts = [torch.randn(32, 48, generator=g) * 0.02 for _ in range(4)]
    bucketed = [nn.Parameter(s.clone().to(DEV)) for s in starts]
    alone = [nn.Parameter(s.clone().to(DEV)) for s in starts]
    together = _dion(bucketed, 1.0)
    separately = [_dion([p], 1.0) for p in alone]
    for _ in range(3):
        for ours, ref in zip(bucketed, alone):
            grad = torch.randn(32, 48, generator=g).to(DEV)
            ours.grad, ref.grad = grad.clone(), grad.clone()
        together.step()
        for opt in separately:
            opt.step()
    assert runs[:2] == [2, 2], runs
    for ours, ref in zip(bucketed, alone):
        torch.testing.assert_close(ours.detach(), ref.detach(), rtol=1e-5, atol=1e-6)


def test_head_split_equals_separate_heads() -> None:
    g = torch.Generator().manual_seed(6)
    start = torch.randn(3 * 64, 128, generator=g) * 0.02
    grad = torch.randn(3 * 64, 128, generator=g)
    fused = nn.Parameter(start.clone().to(DEV))
    opt = _dion([fused], 0.5, heads=3)
    fused.grad = grad.to(DEV)
    opt.step()
    heads = [nn.Parameter(start[i * 64:(i + 1) * 64].clone().to(DEV)) for i in range(3)]
    opt2 = _dion(heads, 0.5)
    for i, h in enumerate(heads):
        h.grad = grad[i * 64:(i + 1) * 64].to(DEV)
    opt2.step()
    assert torch.equal(fused.detach(), torch.cat([h.detach() for h in heads]))


def test_gpu_ema_schedule() -> None:
    torch.manual_seed(7)
    p = nn.Parameter(torch.randn(100, device=DEV))
    opt = Dion([{"params": [p], ROUTE_KEY: "adamw"}], lr=1e-2,
               ema=EMAConfig(decay=0.9, update_every_n_steps=2))
    expected = None
    for step in range(1, 7):
        p.grad = torch.randn_like(p)
        opt.step()
        if step % 2 == 0:
            if expected is None:
                expected = p.detach().clone()
            else:
                expected = torch.lerp(expected, p.detach(), 1 - 0.9**2)
    torch.testing.assert_close(opt.state[p]["ema_shadow"], expected, rtol=1e-6, atol=0)


@pytest.mark.parametrize("nesterov", [False, True])
def test_every_row_run_with_more_tensors_than_one_table(nesterov: bool) -> None:
    """A run of 60 same-shape parameters (more than one 48-entry pointer table)
    on the every-row path: momentum bit-exact, updates as the oracle's."""
    g = torch.Generator().manual_seed(11)
    starts = torch.randn(60, 64, 96, generator=g) * 0.02
    params = [nn.Parameter(s.clone().to(DEV)) for s in starts]
    opt = _dion(params, 1.0, kind=NewtonSchulz.KELLER_TRITON, normuon=not nesterov,
                nesterov=nesterov, weight_decay=0.05)
    grads = torch.randn(60, 64, 96, generator=g) * 1e-3
    for p, gr in zip(params, grads):
        p.grad = gr.to(DEV)
    opt.step()
    w, mom, var = starts.clone(), torch.zeros_like(starts), torch.zeros(60, 64, 1)
    dion_ref.step_blocks(w, grads, mom, var, k=64, lr=LR, mu=0.95, beta2=0.95, weight_decay=0.05,
                         kind="keller_triton", normuon=not nesterov, nesterov=nesterov)
    got_m = torch.stack([opt.state[p]["momentum"].cpu() for p in params])
    assert torch.equal(got_m, mom)
    decay = 1 - LR * 0.05
    got = torch.stack([p.detach().cpu() for p in params])
    assert rel_fro(got - starts * decay, w - starts * decay) < 3e-2


def test_muon_update_matches_oracle() -> None:
    """MUON_UPDATE: Nesterov momentum, Keller quintic, no row normalization."""
    g = torch.Generator().manual_seed(8)
    start = torch.randn(256, 384, generator=g) * 0.02
    param = nn.Parameter(start.clone().to(DEV))
    opt = _dion([param], 1.0, kind=NewtonSchulz.KELLER_TRITON, normuon=False, nesterov=True,
                weight_decay=0.05)
    w = start[None].clone()
    mom = torch.zeros_like(w)
    var = torch.zeros(1, 256, 1)
    for step in range(3):
        grad = torch.randn(256, 384, generator=g) * 1e-3
        param.grad = grad.to(DEV)
        before = param.detach().cpu().clone()
        opt.step()
        w = before[None].clone()
        dion_ref.step_blocks(w, grad[None], mom, var, k=256, lr=LR, mu=0.95, beta2=0.95,
                             weight_decay=0.05, kind="keller_triton", normuon=False, nesterov=True)
        assert torch.equal(opt.state[param]["momentum"].cpu()[None], mom)
        assert rel_fro(param.detach().cpu() - before * (1 - LR * 0.05),
                       w[0] - before * (1 - LR * 0.05)) < 3e-2, f"step {step}"
