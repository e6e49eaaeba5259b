"""Dion's public behaviour on the GPU beyond the numerics: a small model with
every route trains, layouts (conv, channels-last) step like their plain matrix,
groups added late, construction and checkpoint checks (behaviour of
tests/test_optimizer.py:136-168, 200-500, 570-840 of the reference, restated).

microsoft/dion is not available here, so where the reference compares a conv
weight with its NorMuon(flatten=True), this file compares it with the same
weights as one (out, in * k) matrix stepped by this optimizer: bit-exact.
"""

from __future__ import annotations

import copy

import pytest
import torch
from torch import Tensor, nn

import dionw_amd as dionw
import dionw_amd._buckets
from dionw_amd import (
    FRACTION_KEY,
    NEWTON_SCHULZ_KEY,
    NUM_HEADS_KEY,
    ROUTE_KEY,
    Dion,
    MatrixUpdate,
    MomentumForm,
    NewtonSchulz,
    Route,
    RouteKind,
    RowNormalization,
)

pytestmark = pytest.mark.gpu
LR = 1e-3


def _matrix_dion(params, fraction: float = 1.0, kind: NewtonSchulz = NewtonSchulz.GRAM, *,
                 weight_decay: float = 0.0) -> Dion:
    return Dion([{"params": list(params), ROUTE_KEY: "matrix", FRACTION_KEY: fraction}],
                lr=LR, momentum=0.95, muon_beta2=0.95, betas=(0.9, 0.99),
                weight_decay=weight_decay, eps=1e-8,
                matrix_update=MatrixUpdate(newton_schulz=kind,
                                           row_normalization=RowNormalization.NORMUON,
                                           momentum_form=MomentumForm.HEAVY_BALL))


def _polar(x: Tensor, eps: float) -> Tensor:
    """Exact polar factor (float64 SVD): keeps Newton-Schulz rounding out of
    comparisons between layouts."""
    del eps
    u, _, vh = torch.linalg.svd(x.double(), full_matrices=False)
    return (u @ vh).to(torch.bfloat16)


def _rand(shape, gen: torch.Generator) -> Tensor:
    return torch.randn(*shape, generator=gen).cuda()


class _Tiny(nn.Module):
    """A small model touching every route: an embedding, a fused q/k/v split
    into heads, a conv, a feed-forward pair, a norm, a learned token and a
    narrow output."""

    def __init__(self) -> None:
        super().__init__()
        self.embed = nn.Embedding(16, 48)
        self.qkv = nn.Linear(48, 144)
        self.mix = nn.Conv1d(48, 48, 5, padding=2)
        self.ff_in = nn.Linear(48, 96)
        self.ff_out = nn.Linear(96, 48)
        self.ln = nn.LayerNorm(48)
        self.out = nn.Linear(48, 4)
        self.cls_token = nn.Parameter(torch.zeros(1, 1, 48))

    def dion_routes(self):
        yield self.qkv.weight, Route(RouteKind.MATRIX, num_heads=12)

    def forward(self, ids: Tensor) -> Tensor:
        x = self.embed(ids) + self.cls_token
        q, k, v = self.qkv(x).chunk(3, dim=-1)
        x = x + q * torch.sigmoid(k) + 0.1 * v
        x = x + self.mix(x.mT).mT
        x = x + self.ff_out(nn.functional.gelu(self.ff_in(self.ln(x))))
        return self.out(x)


def _tiny_dion(model: nn.Module, lr: float, kind: NewtonSchulz) -> Dion:
    groups, _ = dionw.param_groups(model, fraction=0.5, selection_min_dim=32, min_matrix_dim=8)
    return Dion(groups, lr=lr, momentum=0.95, muon_beta2=0.95, betas=(0.9, 0.98),
                weight_decay=0.01, eps=1e-8,
                matrix_update=MatrixUpdate(newton_schulz=kind,
                                           row_normalization=RowNormalization.NORMUON,
                                           momentum_form=MomentumForm.HEAVY_BALL))


@pytest.mark.parametrize("kind", list(NewtonSchulz))
def test_tiny_model_trains(kind: NewtonSchulz) -> None:
    torch.manual_seed(0)
    model = _Tiny().cuda()
    opt = _tiny_dion(model, 1e-2, kind)
    gen = torch.Generator().manual_seed(0)
    ids = torch.randint(0, 16, (8, 12), generator=gen).cuda()
    target = torch.randn(8, 12, 4, generator=gen).cuda()
    losses = []
    for _ in range(30):
        loss = (model(ids) - target).pow(2).mean()
        losses.append(float(loss.detach()))
        loss.backward()
        opt.step()
        opt.zero_grad(set_to_none=True)
    assert losses[-1] < 0.75 * losses[0], losses


def test_zero_lr_freezes_every_route() -> None:
    torch.manual_seed(0)
    model = _Tiny().cuda()
    opt = _tiny_dion(model, 0.0, NewtonSchulz.GRAM)
    before = {n: p.detach().clone() for n, p in model.named_parameters()}
    gen = torch.Generator().manual_seed(1)
    for _ in range(2):
        for p in model.parameters():
            p.grad = _rand(p.shape, gen)
        opt.step()
    for n, p in model.named_parameters():
        assert torch.equal(p.detach(), before[n]), n


def test_weights_without_gradients_stay_put() -> None:
    gen = torch.Generator().manual_seed(0)
    weights = [nn.Parameter(_rand((32, 32), gen)) for _ in range(3)]
    opt = _matrix_dion(weights, 0.5)
    untouched = weights[1].detach().clone()
    first = weights[0].detach().clone()
    weights[0].grad = _rand((32, 32), gen)
    weights[2].grad = _rand((32, 32), gen)
    opt.step()
    assert torch.equal(weights[1].detach(), untouched)
    assert not torch.equal(weights[0].detach(), first)


@pytest.mark.parametrize("weight_decay", [0.0, 0.1])
def test_conv_weight_steps_as_its_flattened_matrix(weight_decay: float,
                                                   monkeypatch: pytest.MonkeyPatch) -> None:
    """A (out, in, k) conv weight is the (out, in * k) matrix (_buckets.py:75-90)."""
    monkeypatch.setattr(dionw_amd._buckets, "newton_schulz_fn", lambda _kind: _polar)
    gen = torch.Generator().manual_seed(0)
    start = _rand((32, 16, 3), gen) * 0.02
    conv = nn.Parameter(start.clone())
    flat = nn.Parameter(start.reshape(32, 48).clone())
    opts = [_matrix_dion([p], 1.0, NewtonSchulz.POLAR_EXPRESS, weight_decay=weight_decay)
            for p in (conv, flat)]
    for _ in range(4):
        g = _rand((32, 16, 3), gen)
        conv.grad, flat.grad = g.clone(), g.reshape(32, 48).clone()
        for opt in opts:
            opt.step()
    assert torch.equal(conv.detach().reshape(32, 48), flat.detach())


@pytest.mark.parametrize("fraction", [0.5, 1.0])
def test_channels_last_conv_steps_like_contiguous(fraction: float) -> None:
    torch.manual_seed(0)
    plain = nn.Conv2d(32, 64, 3).cuda()
    strided = nn.Conv2d(32, 64, 3).cuda()
    strided.weight.data = strided.weight.data.contiguous(memory_format=torch.channels_last)
    strided.load_state_dict(plain.state_dict())
    assert not strided.weight.is_contiguous()
    opts = [_matrix_dion([c.weight], fraction) for c in (plain, strided)]
    gen = torch.Generator().manual_seed(1)
    for _ in range(3):
        g = _rand(plain.weight.shape, gen)
        plain.weight.grad = g.clone()
        strided.weight.grad = g.clone().contiguous(memory_format=torch.channels_last)
        for opt in opts:
            opt.step()
    assert not strided.weight.is_contiguous()
    torch.testing.assert_close(strided.weight, plain.weight, rtol=0, atol=1e-6)


def test_group_added_after_a_step_is_stepped() -> None:
    gen = torch.Generator().manual_seed(0)
    first = nn.Parameter(_rand((32, 32), gen))
    second = nn.Parameter(_rand((32, 32), gen))
    opt = _matrix_dion([first])
    first.grad = _rand((32, 32), gen)
    opt.step()
    momentum = opt.state[first]["momentum"].clone()
    with pytest.raises(ValueError, match="fraction"):
        opt.add_param_group({"params": [second], ROUTE_KEY: "matrix", FRACTION_KEY: 1.5})
    assert len(opt.param_groups) == 1
    opt.add_param_group({"params": iter([second]), ROUTE_KEY: "matrix", FRACTION_KEY: 1.0})
    before = second.detach().clone()
    first.grad = None
    second.grad = _rand((32, 32), gen)
    opt.step()
    assert not torch.equal(second.detach(), before)
    # The repacked bucket kept the first weight's momentum.
    assert torch.equal(opt.state[first]["momentum"], momentum)


def test_construction_errors() -> None:
    w = nn.Parameter(torch.zeros(16, 16, device="cuda"))
    with pytest.raises(TypeError, match=r"dionw\.param_groups"):
        Dion([w], lr=LR)
    with pytest.raises(ValueError, match="CUDA"):
        _matrix_dion([nn.Parameter(torch.zeros(16, 16))])
    with pytest.raises(TypeError, match="float32 parameters"):
        _matrix_dion([w.detach().bfloat16().requires_grad_()])
    with pytest.raises(ValueError, match="momentum"):
        Dion([{"params": [w], ROUTE_KEY: "matrix"}], lr=LR, momentum=1.0)


def test_checkpoint_without_newton_schulz_kind_is_refused() -> None:
    w = nn.Parameter(torch.zeros(16, 16, device="cuda"))
    opt = _matrix_dion([w])
    state = opt.state_dict()
    del state["param_groups"][0][NEWTON_SCHULZ_KEY]
    with pytest.raises(ValueError, match=NEWTON_SCHULZ_KEY):
        opt.load_state_dict(state)


def test_checkpoint_from_before_the_update_options_resumes_only_as_normuon() -> None:
    """A checkpoint whose groups lack the row-normalization and momentum-form
    keys is NorMuon with heavy-ball momentum: it resumes into that optimizer
    (the next step bit-equal to the uninterrupted one) and is refused by a
    Muon (reference tests/test_muon.py:318-342)."""
    gen = torch.Generator().manual_seed(5)
    w = nn.Parameter(_rand((64, 48), gen))
    opt = _matrix_dion([w])
    w.grad = _rand((64, 48), gen)
    opt.step()
    state = copy.deepcopy(opt.state_dict())
    for group in state["param_groups"]:
        del group["row_normalization"], group["momentum_form"]
    twin = nn.Parameter(w.detach().clone())
    resumed = _matrix_dion([twin])
    resumed.load_state_dict(copy.deepcopy(state))
    assert resumed.param_groups[0]["row_normalization"] == "normuon"
    assert resumed.param_groups[0]["momentum_form"] == "heavy_ball"
    grad = _rand((64, 48), gen)
    w.grad, twin.grad = grad.clone(), grad.clone()
    opt.step()
    resumed.step()
    assert torch.equal(twin.detach(), w.detach())
    muon = Dion([{"params": [nn.Parameter(w.detach().clone())], ROUTE_KEY: "matrix",
                  FRACTION_KEY: 1.0}], lr=LR, momentum=0.95, muon_beta2=0.95,
                betas=(0.9, 0.99), weight_decay=0.0, eps=1e-8,
                matrix_update=MatrixUpdate(NewtonSchulz.GRAM, RowNormalization.NONE,
                                           MomentumForm.HEAVY_BALL))
    with pytest.raises(ValueError, match="'row_normalization'"):
        muon.load_state_dict(copy.deepcopy(state))


def test_saved_state_keeps_one_storage_per_bucket(tmp_path) -> None:
    gen = torch.Generator().manual_seed(0)
    weights = [nn.Parameter(_rand((32, 32), gen)) for _ in range(2)]
    opt = _matrix_dion(weights)
    for w in weights:
        w.grad = _rand((32, 32), gen)
    opt.step()
    path = tmp_path / "state.pt"
    torch.save(opt.state_dict(), path)
    loaded = torch.load(path, weights_only=True)
    a, b = (loaded["state"][i]["momentum"] for i in (0, 1))
    assert a.untyped_storage().data_ptr() == b.untyped_storage().data_ptr()
    assert a.untyped_storage().nbytes() == 2 * 32 * 32 * 4


def test_decay_reaches_every_row_and_spares_exempt_groups() -> None:
    gen = torch.Generator().manual_seed(0)
    decayed = nn.Parameter(_rand((64, 96), gen))
    exempt = nn.Parameter(_rand((64, 96), gen))
    start = [decayed.detach().clone(), exempt.detach().clone()]
    opt = Dion([{"params": [decayed], ROUTE_KEY: "matrix", FRACTION_KEY: 0.5},
                {"params": [exempt], ROUTE_KEY: "matrix", FRACTION_KEY: 0.5,
                 "weight_decay": 0.0}],
               lr=LR, momentum=0.95, muon_beta2=0.95, weight_decay=0.1)
    decayed.grad, exempt.grad = torch.zeros_like(decayed), torch.zeros_like(exempt)
    opt.step()
    decay = torch.tensor(1 - LR * 0.1, dtype=torch.float32)
    assert torch.equal(decayed.detach(), start[0] * decay.cuda())
    assert torch.equal(exempt.detach(), start[1])


@pytest.mark.parametrize("fraction", [0.25, 1.0])
def test_plugged_in_orthogonalization_receives_float32(fraction: float,
                                                       monkeypatch: pytest.MonkeyPatch) -> None:
    """A plugged-in Newton-Schulz gets the unrounded float32 momentum (the
    selected rows at fraction 0.25, the full block at 1.0)."""
    seen: list[tuple[torch.dtype, tuple[int, ...]]] = []

    def recording(x: Tensor, eps: float) -> Tensor:
        seen.append((x.dtype, tuple(x.shape)))
        return _polar(x, eps)

    monkeypatch.setattr(dionw_amd._buckets, "newton_schulz_fn", lambda _kind: recording)
    gen = torch.Generator().manual_seed(0)
    w = nn.Parameter(_rand((64, 128), gen))
    w.grad = _rand((64, 128), gen)
    _matrix_dion([w], fraction).step()
    assert seen == [(torch.float32, (1, int(64 * fraction), 128))]


def test_state_before_the_first_step_and_late_adamw_group() -> None:
    gen = torch.Generator().manual_seed(0)
    matrix = nn.Parameter(_rand((32, 32), gen))
    vector = nn.Parameter(_rand((32,), gen))
    opt = _matrix_dion([matrix])
    opt.initialize_state(matrix)
    assert not opt.state[matrix]["momentum"].any()
    with pytest.raises(ValueError, match="not in the optimizer"):
        opt.initialize_state(vector)
    opt.add_param_group({"params": [vector], ROUTE_KEY: "adamw"})
    assert not opt.state[vector]["exp_avg"].any()
    before = vector.detach().clone()
    vector.grad = _rand((32,), gen)
    opt.step()
    assert not torch.equal(vector.detach(), before)


def test_groups_checked_when_added() -> None:
    w = nn.Parameter(torch.zeros(30, 16, device="cuda"))
    with pytest.raises(ValueError, match="does not divide"):
        _matrix_dion([w]).add_param_group(
            {"params": [nn.Parameter(torch.zeros(30, 16, device="cuda"))],
             ROUTE_KEY: "matrix", NUM_HEADS_KEY: 4})
    with pytest.raises(ValueError, match="route it to AdamW"):
        _matrix_dion([nn.Parameter(torch.zeros(16, device="cuda"))])
    with pytest.raises(ValueError, match="lr and weight_decay"):
        _matrix_dion([w]).add_param_group(
            {"params": [nn.Parameter(torch.zeros(8, 8, device="cuda"))], ROUTE_KEY: "matrix",
             "lr": -1.0})


@pytest.mark.parametrize(("key", "value"), [
    ("fraction", 0.25),
    ("newton_schulz", NewtonSchulz.POLAR_EXPRESS.value),
    ("dion_route", "adamw"),
    ("row_normalization", RowNormalization.NONE.value),
    ("momentum_form", MomentumForm.NESTEROV.value),
])
def test_structurally_different_checkpoint_is_refused(key: str, value: object) -> None:
    gen = torch.Generator().manual_seed(0)
    w = nn.Parameter(_rand((32, 32), gen))
    opt = _matrix_dion([w], 0.5)
    w.grad = _rand((32, 32), gen)
    opt.step()
    state = copy.deepcopy(opt.state_dict())
    state["param_groups"][0][key] = value
    with pytest.raises(ValueError, match=f"'{key}'"):
        opt.load_state_dict(state)
