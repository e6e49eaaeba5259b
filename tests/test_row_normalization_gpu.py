"""The ``finish`` / ``normalize_rows`` seam on the HIP library (GPU).

Reference interface: src/dionw/_row_normalization.py:18-60. Two bars:
- against the float64 closed form (within 2e-6) and the oracle's CPU
  restatement of ``normalize_rows`` (float32 torch ops, another summation
  order: no further than the oracle's own rounding allows);
- against the optimizer's fused step: the weights a ``Dion.step`` writes equal
  ``W * decay + finish(O, v, group, step)`` bit for bit, where ``O`` is the
  Newton-Schulz output the step itself produced (recorded through the
  replaceable ``newton_schulz_fn``), and the step's new variance equals the
  seam's.
"""

from __future__ import annotations

import math

import pytest
import torch
from torch import nn

import dionw_amd._buckets
from dionw_amd import (
    FRACTION_KEY,
    ROUTE_KEY,
    Dion,
    MatrixUpdate,
    MomentumForm,
    NewtonSchulz,
    RowNormalization,
)
from dionw_amd._keys import MUON_BETA2_KEY, ROW_NORMALIZATION_KEY
from dionw_amd._row_normalization import finish, normalize_rows
from dionw_amd.newton_schulz import newton_schulz_fn
from oracle import dion_ref
from tests.conftest import rel_fro

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _normalize_rows_float64(o: torch.Tensor, variance: torch.Tensor, beta2: float,
                            step: float) -> torch.Tensor:
    """NorMuon in float64 (no rounding), the closed form both are measured against."""
    u, v = o.double(), variance.double()
    v = v + (u.square().mean(-1, keepdim=True) - v) * (1.0 - beta2)
    n = u / (v.sqrt() + 1e-8)
    new_norm = n.norm(dim=(-2, -1), keepdim=True).clamp_min(1e-8)
    restore = u.norm(dim=(-2, -1), keepdim=True) / new_norm
    return n * (restore * step)


@pytest.mark.parametrize(("blocks", "k", "cols"), [(1, 64, 256), (3, 100, 70), (2, 1024, 4096),
                                                   (4, 352, 2048), (1, 5, 3)])
def test_normalize_rows_matches_the_oracle(blocks: int, k: int, cols: int) -> None:
    """The float32 step within 2e-6 of the float64 closed form, and no further
    from the oracle than the oracle's own rounding allows: torch's CPU float32
    norms over a whole block round by up to ~1e-4 at 4 M elements, where the
    kernels' per-row and per-block tree sums stay near 1e-7."""
    g = torch.Generator().manual_seed(blocks * 1000 + k)
    o = (torch.randn(blocks, k, cols, generator=g) / math.sqrt(cols)).bfloat16()
    variance = torch.rand(blocks, k, 1, generator=g) * 1e-3 / cols
    variance[:, ::3] = 0.0  # fresh rows next to used ones
    step = torch.tensor(-3.7e-3)
    want_delta, want_v = dion_ref.normalize_rows(o, variance, 0.95, step)
    exact = _normalize_rows_float64(o, variance, 0.95, float(step))
    v_dev = variance.to(DEV)
    got_delta, got_v = normalize_rows(o.to(DEV), v_dev, 0.95, step.to(DEV))
    assert torch.equal(v_dev.cpu(), variance), "the input variance must not change"
    assert got_delta.dtype == torch.float32 and got_delta.shape == (blocks, k, cols)
    assert got_v.shape == (blocks, k, 1)
    case = f"{blocks}x{k}x{cols}"
    assert rel_fro(got_v.cpu(), want_v) < 1e-6, f"{case}: variance"
    gpu_err = rel_fro(got_delta.cpu(), exact)
    assert gpu_err < 2e-6, f"{case}: step {gpu_err} from the float64 closed form"
    oracle_err = rel_fro(want_delta, exact)
    assert rel_fro(got_delta.cpu(), want_delta) < oracle_err + 2e-6, (
        f"{case}: step vs oracle (oracle rounding {oracle_err})")


def test_finish_without_normalization_is_the_scaled_output() -> None:
    g = torch.Generator().manual_seed(7)
    o = torch.randn(2, 48, 96, generator=g).bfloat16()
    group = {ROW_NORMALIZATION_KEY: RowNormalization.NONE.value, MUON_BETA2_KEY: 0.95}
    delta, v = finish(o.to(DEV), torch.zeros(2, 48, 1, device=DEV), group,
                      torch.tensor(-0.25, device=DEV))
    assert v is None
    assert torch.equal(delta.cpu(), o.float() * torch.tensor(-0.25))


def test_finish_rejects_bad_arguments() -> None:
    o = torch.zeros(2, 8, 16, device=DEV, dtype=torch.bfloat16)
    group = {ROW_NORMALIZATION_KEY: RowNormalization.NORMUON.value, MUON_BETA2_KEY: 0.95}
    with pytest.raises(ValueError, match="variance"):
        finish(o, torch.zeros(2, 8, device=DEV), group, -1.0)
    with pytest.raises(ValueError, match="blocks, k, cols"):
        finish(o[0], torch.zeros(8, 1, device=DEV), group, -1.0)
    with pytest.raises(ValueError, match="GPU"):
        finish(o.cpu(), torch.zeros(2, 8, 1), group, -1.0)


@pytest.mark.parametrize(("shape", "fraction", "weight_decay"),
                         [((512, 1024), 1.0, 0.05), ((768, 512), 0.25, 0.0),
                          ((1024, 4096), 0.25, 0.0)])
def test_finish_equals_the_fused_step(monkeypatch, shape, fraction, weight_decay) -> None:
    """The fused step adds exactly the seam's step to ``W * decay``."""
    recorded = []
    real = newton_schulz_fn(NewtonSchulz.GRAM)

    def recording(x: torch.Tensor, epsilon: float) -> torch.Tensor:
        out = real(x, epsilon)
        recorded.append(out.clone())
        return out

    monkeypatch.setattr(dionw_amd._buckets, "newton_schulz_fn", lambda kind: recording)
    g = torch.Generator().manual_seed(11)
    lr = 2e-3
    param = nn.Parameter((torch.randn(*shape, generator=g) * 0.02).to(DEV))
    opt = Dion([{"params": [param], ROUTE_KEY: "matrix", FRACTION_KEY: fraction}], lr=lr,
               momentum=0.95, muon_beta2=0.95, weight_decay=weight_decay,
               matrix_update=MatrixUpdate(NewtonSchulz.GRAM, RowNormalization.NORMUON,
                                          MomentumForm.HEAVY_BALL))
    rows, cols = shape
    k = min(rows, math.ceil(fraction * rows))
    step = -lr * 0.2 * math.sqrt(max(rows, cols)) * math.sqrt(min(rows, cols) / min(k, cols))
    for it in range(2):
        param.grad = (torch.randn(*shape, generator=g) * 1e-3).to(DEV)
        before = param.detach().clone()
        var_before = (opt.state[param]["variance"].clone() if it
                      else torch.zeros(rows, 1, device=DEV))
        recorded.clear()
        opt.step()
        torch.cuda.synchronize()
        (o,) = recorded
        var_after = opt.state[param]["variance"]
        if fraction == 1.0:
            idx = torch.arange(rows, device=DEV)
        else:
            # Only the selected rows' variance moves (weight decay off: only
            # they move in W as well); they are stored in ascending row order.
            idx = torch.nonzero((var_after != var_before).view(-1)).view(-1)
            assert idx.numel() == k, f"step {it}: {idx.numel()} rows changed, expected {k}"
        group = opt.param_groups[0]
        delta, v_new = finish(o.view(1, k, cols), var_before[idx].view(1, k, 1), group,
                              torch.tensor(step, dtype=torch.float32, device=DEV))
        decay = torch.tensor(1.0 - lr * weight_decay, dtype=torch.float32)
        expected = before * decay if weight_decay > 0 else before.clone()
        expected[idx] = expected[idx] + delta[0]
        assert torch.equal(param.detach(), expected), f"step {it}: weights differ from W d + step"
        assert torch.equal(var_after[idx].view(-1), v_new.view(-1)), f"step {it}: variance"
