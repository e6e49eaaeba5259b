"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_fixtures.py).

CPU: the oracle still reproduces them (bit-exact for scores, indices and
momentum). GPU: the HIP step reproduces them — exact polar factor: weights to
float32 rounding; the 1024x1024 NorMuon step of config1.npz: the whole update
within 1e-2 relative Frobenius, variance within 2e-2, momentum exact.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
from torch import nn

from tests.golden import make_fixtures as fx

GOLDEN = fx.HERE


def _load(name: str) -> dict:
    with np.load(GOLDEN / name, allow_pickle=False) as data:
        return {k: data[k] for k in data.files}


def test_oracle_reproduces_small_fixture() -> None:
    want = _load("small_step.npz")
    got = fx.small_expected()
    for key in want:
        if key.startswith(("scores", "index", "momentum")):
            assert np.array_equal(got[key], want[key]), key
        else:
            np.testing.assert_allclose(got[key], want[key], rtol=0, atol=1e-7, err_msg=key)


def test_oracle_reproduces_config1_fixture() -> None:
    want = _load("config1.npz")
    got = fx.config1_expected()
    assert got["momentum_abs_sum"] == want["momentum_abs_sum"]
    np.testing.assert_allclose(got["weight_corner"], want["weight_corner"], rtol=0, atol=1e-7)
    np.testing.assert_allclose(got["update_norm"], want["update_norm"], rtol=1e-6)
    assert np.array_equal(got["update_f16"], want["update_f16"])
    assert got["update_scale"] == want["update_scale"]


def _fixture_update(want: dict) -> np.ndarray:
    return want["update_f16"].astype(np.float64) * float(want["update_scale"])


@pytest.mark.gpu
def test_hip_step_matches_small_fixture(monkeypatch) -> None:
    import dionw_amd._buckets
    from dionw_amd import Dion

    monkeypatch.setattr(
        dionw_amd._buckets,
        "newton_schulz_fn",
        lambda _kind: lambda x, eps: fx.exact_polar(x.cpu(), eps).to(x.device),
    )
    want = _load("small_step.npz")
    w, grads = fx.small_inputs()
    params = [nn.Parameter(w[i].clone().cuda()) for i in range(2)]
    opt = Dion([{"params": params, "dion_route": "matrix", "fraction": 0.25}], lr=1e-3,
               momentum=0.95, muon_beta2=0.95, weight_decay=0.1)
    for step in range(3):
        for i, p in enumerate(params):
            p.grad = grads[step, i].cuda()
        opt.step()
        mom = np.stack([opt.state[p]["momentum"].cpu().numpy() for p in params])
        assert np.array_equal(mom, want[f"momentum{step}"]), f"step {step}: momentum"
        weights = np.stack([p.detach().cpu().numpy() for p in params])
        np.testing.assert_allclose(weights, want[f"weight{step}"], rtol=0, atol=2e-7,
                                   err_msg=f"step {step}: weights")
        var = np.stack([opt.state[p]["variance"].cpu().numpy() for p in params])
        np.testing.assert_allclose(var, want[f"variance{step}"], rtol=1e-5, atol=1e-12)


@pytest.mark.gpu
def test_hip_step_matches_config1_fixture() -> None:
    from dionw_amd import Dion

    want = _load("config1.npz")
    w, grad = fx.config1_inputs()
    p = nn.Parameter(w.clone().cuda())
    opt = Dion([{"params": [p], "dion_route": "matrix", "fraction": 1.0}], lr=3e-4,
               momentum=0.95, muon_beta2=0.95, weight_decay=0.05)
    p.grad = grad.cuda()
    opt.step()
    got = p.detach().cpu()
    update = got - w * (1.0 - 3e-4 * 0.05)
    assert abs(float(update.double().norm()) - float(want["update_norm"])) < 1e-2 * float(
        want["update_norm"]
    )
    corner_ref = want["weight_corner"] - w[:64, :64].numpy() * (1.0 - 3e-4 * 0.05)
    corner_got = update[:64, :64].numpy()
    rel = np.linalg.norm(corner_got - corner_ref) / np.linalg.norm(corner_ref)
    assert rel < 2e-2, rel
    whole_ref = _fixture_update(want)
    rel_whole = np.linalg.norm(update.double().numpy() - whole_ref) / np.linalg.norm(whole_ref)
    assert rel_whole < 1e-2, rel_whole
    var = opt.state[p]["variance"].cpu().numpy()[:, 0]
    rel_v = np.linalg.norm(var - want["variance"]) / np.linalg.norm(want["variance"])
    assert rel_v < 2e-2, rel_v
    assert math.isclose(float(opt.state[p]["momentum"].double().abs().sum()),
                        float(want["momentum_abs_sum"]), rel_tol=0, abs_tol=0)
