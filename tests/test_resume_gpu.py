"""Checkpoints at the BASELINE configurations' scale (GPU).

Restates the reference's resume, storage and repacking tests
(tests/test_optimizer.py:309-374, 417-453, 481-494) at GPT-2-small scale
(config 3, 124 M parameters) and MoE scale (config 5a, 553 M parameters,
GPU EMA), and loads a state dict laid out by the reference's key contract
(src/dionw/_keys.py:33-68, ema/_keys.py) written without this package's
``state_dict``.
"""

from __future__ import annotations

import io

import pytest
import torch
from torch import nn

from dionw_amd import FRACTION_KEY, ROUTE_KEY, Dion, EMAConfig

pytestmark = pytest.mark.gpu
DEV = "cuda"
LR, WD = 3e-4, 0.05


def _say(msg: str) -> None:
    print(f"[resume] {msg}", flush=True)


def _gpt2_params(seed: int) -> tuple[list[nn.Parameter], list[nn.Parameter]]:
    g = torch.Generator(device=DEV).manual_seed(seed)

    def p(*shape):
        return nn.Parameter(torch.empty(*shape, device=DEV).normal_(0, 0.02, generator=g))

    mats = [p(r, c) for _ in range(12) for r, c in ((2304, 768), (768, 768), (3072, 768),
                                                     (768, 3072))]
    vecs = [p(50257, 768), p(1024, 768)] + [p(n) for n in [2304, 768, 3072, 768] * 12]
    return mats, vecs


def _gpt2_opt(mats, vecs, ema) -> Dion:
    return Dion([{"params": mats, ROUTE_KEY: "matrix", FRACTION_KEY: 1.0},
                 {"params": vecs, ROUTE_KEY: "adamw"}],
                lr=LR, weight_decay=WD, ema=ema)


def _grads(params, seed: int) -> None:
    g = torch.Generator(device=DEV).manual_seed(seed)
    for p in params:
        p.grad = torch.empty_like(p).normal_(0, 1e-3, generator=g)


def _assert_same(opt_a: Dion, params_a, opt_b: Dion, params_b, what: str) -> None:
    for i, (a, b) in enumerate(zip(params_a, params_b, strict=True)):
        assert torch.equal(a.detach(), b.detach()), f"{what}: parameter {i}"
        sa, sb = opt_a.state[a], opt_b.state[b]
        assert sa.keys() == sb.keys(), f"{what}: state keys of {i}"
        for key, value in sa.items():
            if isinstance(value, torch.Tensor):
                assert torch.equal(value, sb[key].to(value.device)), f"{what}: {key} of {i}"


def _save_load(opt: Dion) -> dict:
    buf = io.BytesIO()
    torch.save(opt.state_dict(), buf)
    buf.seek(0)
    return torch.load(buf, weights_only=True)


def test_gpt2_resume_is_bit_exact_with_shared_bucket_storage() -> None:
    """Config 3 with a GPU EMA: 2 steps, save, load into fresh parameters and a
    fresh optimizer, 2 more steps equals 4 uninterrupted steps bit for bit
    (weights, momentum, variance, AdamW moments and counters, EMA shadows).
    The saved momenta of each bucket share one storage of the bucket's size."""
    _say("GPT-2 small: uninterrupted 4 steps")
    ema = EMAConfig(decay=0.99, update_every_n_steps=1)
    mats, vecs = _gpt2_params(0)
    full = _gpt2_opt(mats, vecs, ema)
    for step in range(4):
        _grads(mats + vecs, 100 + step)
        full.step()
    _say("GPT-2 small: 2 steps, save, load, 2 steps")
    mats1, vecs1 = _gpt2_params(0)
    first = _gpt2_opt(mats1, vecs1, ema)
    for step in range(2):
        _grads(mats1 + vecs1, 100 + step)
        first.step()
    saved = _save_load(first)
    weights = [p.detach().clone() for p in mats1 + vecs1]
    storages: dict[int, list[torch.Tensor]] = {}
    for index in range(48):
        m = saved["state"][index]["momentum"]
        storages.setdefault(m.untyped_storage().data_ptr(), []).append(m)
    assert len(storages) == 4, "one momentum storage per (rows, cols) bucket"
    for views in storages.values():
        assert len(views) == 12
        assert views[0].untyped_storage().nbytes() == 12 * views[0].numel() * 4
    mats2, vecs2 = _gpt2_params(7)  # other values: everything comes from the checkpoint
    with torch.no_grad():
        for p, w in zip(mats2 + vecs2, weights):
            p.copy_(w)
    resumed = _gpt2_opt(mats2, vecs2, ema)
    resumed.load_state_dict(saved)
    for step in range(2, 4):
        _grads(mats2 + vecs2, 100 + step)
        resumed.step()
    full.ema.flush_pending_updates()
    resumed.ema.flush_pending_updates()
    _assert_same(full, mats + vecs, resumed, mats2 + vecs2, "GPT-2 resume")
    assert resumed.state_dict()["_ema_step_count"] == 4


def _experts(seed: int, n: int = 64) -> list[nn.Parameter]:
    g = torch.Generator(device=DEV).manual_seed(seed)
    out = []
    for _ in range(n):
        for r, c in ((1408, 2048), (1408, 2048), (2048, 1408)):
            out.append(nn.Parameter(torch.empty(r, c, device=DEV).normal_(0, 0.02, generator=g)))
    return out


def test_moe_resume_is_bit_exact() -> None:
    """Config 5a (64 experts, f = 0.25, GPU EMA 0.9999): resume after 2 steps
    equals 4 uninterrupted steps bit for bit, selection included."""
    ema = EMAConfig(decay=0.9999, update_every_n_steps=1)
    _say("MoE: uninterrupted 4 steps")
    experts = _experts(0)
    full = Dion([{"params": experts, ROUTE_KEY: "matrix", FRACTION_KEY: 0.25}], lr=LR,
                weight_decay=WD, ema=ema)
    for step in range(4):
        _grads(experts, 200 + step)
        full.step()
    _say("MoE: 2 steps, save, load, 2 steps")
    first_params = _experts(0)
    first = Dion([{"params": first_params, ROUTE_KEY: "matrix", FRACTION_KEY: 0.25}], lr=LR,
                 weight_decay=WD, ema=ema)
    for step in range(2):
        _grads(first_params, 200 + step)
        first.step()
    saved = _save_load(first)
    weights = [p.detach().clone() for p in first_params]
    del first, first_params
    resumed_params = _experts(5)
    with torch.no_grad():
        for p, w in zip(resumed_params, weights):
            p.copy_(w)
    del weights
    resumed = Dion([{"params": resumed_params, ROUTE_KEY: "matrix", FRACTION_KEY: 0.25}],
                   lr=LR, weight_decay=WD, ema=ema)
    resumed.load_state_dict(saved)
    del saved
    for step in range(2, 4):
        _grads(resumed_params, 200 + step)
        resumed.step()
    full.ema.flush_pending_updates()
    resumed.ema.flush_pending_updates()
    _assert_same(full, experts, resumed, resumed_params, "MoE resume")


def test_moe_group_added_after_steps_is_repacked() -> None:
    """Config 5a's gate/up experts step twice; the down experts join as a new
    group: the existing momenta survive the repacking bit for bit, the new
    group steps, and a group with a bad fraction is refused unadded."""
    _say("MoE: add_param_group after 2 steps")
    experts = _experts(0, 16)
    gate_up = [p for i, p in enumerate(experts) if i % 3 != 2]
    down = experts[2::3]
    opt = Dion([{"params": gate_up, ROUTE_KEY: "matrix", FRACTION_KEY: 0.25}], lr=LR,
               weight_decay=WD)
    for step in range(2):
        _grads(gate_up, 300 + step)
        opt.step()
    kept = [opt.state[p]["momentum"].clone() for p in gate_up]
    with pytest.raises(ValueError, match="fraction"):
        opt.add_param_group({"params": down, ROUTE_KEY: "matrix", FRACTION_KEY: 1.5})
    assert len(opt.param_groups) == 1
    opt.add_param_group({"params": iter(down), ROUTE_KEY: "matrix", FRACTION_KEY: 0.25})
    before = [p.detach().clone() for p in down]
    for p in gate_up:
        p.grad = None
    _grads(down, 302)
    opt.step()
    for p, m in zip(gate_up, kept):
        assert torch.equal(opt.state[p]["momentum"], m), "momentum lost in the repacking"
    for p, b in zip(down, before):
        assert not torch.equal(p.detach(), b), "the added group did not step"


def test_state_dict_in_the_reference_layout_loads() -> None:
    """A checkpoint assembled by hand in the reference's layout — group keys
    (dion_route, fraction, num_heads, newton_schulz, row_normalization,
    momentum_form, momentum, muon_beta2 and torch's), per-parameter momentum
    [rows, cols] and variance [rows, 1] as views of one bucket tensor, AdamW
    exp_avg / exp_avg_sq / adamw_step (0-d float32), EMA ema_shadow /
    ema_initialized and the top-level _ema_step_count — resumes exactly like
    this package's own checkpoint, and this package writes exactly those keys."""
    ema = EMAConfig(decay=0.9, update_every_n_steps=1)
    g = torch.Generator(device=DEV).manual_seed(4)

    def params():
        mats = [nn.Parameter(torch.randn(256, 512, generator=g, device=DEV) * 0.02)
                for _ in range(2)]
        return mats, [nn.Parameter(torch.randn(512, generator=g, device=DEV) * 0.02)]

    def opt(mats, vecs):
        return Dion([{"params": mats, ROUTE_KEY: "matrix", FRACTION_KEY: 0.5},
                     {"params": vecs, ROUTE_KEY: "adamw", "weight_decay": 0.0}],
                    lr=1e-3, weight_decay=WD, ema=ema)

    mats, vecs = params()
    source = opt(mats, vecs)
    for step in range(2):
        _grads(mats + vecs, 400 + step)
        source.step()
    own = source.state_dict()
    group_keys = {"params", "lr", "betas", "eps", "weight_decay", "momentum", "muon_beta2",
                  "fraction", "num_heads", "newton_schulz", "row_normalization",
                  "momentum_form", "dion_route"}
    assert all(set(grp) == group_keys for grp in own["param_groups"])
    assert set(own["state"][0]) == {"momentum", "variance", "ema_shadow", "ema_initialized"}
    assert set(own["state"][2]) == {"exp_avg", "exp_avg_sq", "adamw_step", "ema_shadow",
                                    "ema_initialized"}
    bucket_m = torch.stack([source.state[p]["momentum"] for p in mats]).cpu()
    bucket_v = torch.stack([source.state[p]["variance"] for p in mats]).cpu()
    vec_state = source.state[vecs[0]]
    layout = {
        "state": {
            0: {"momentum": bucket_m[0], "variance": bucket_v[0],
                "ema_shadow": source.state[mats[0]]["ema_shadow"].cpu(), "ema_initialized": True},
            1: {"momentum": bucket_m[1], "variance": bucket_v[1],
                "ema_shadow": source.state[mats[1]]["ema_shadow"].cpu(), "ema_initialized": True},
            2: {"exp_avg": vec_state["exp_avg"].cpu(), "exp_avg_sq": vec_state["exp_avg_sq"].cpu(),
                "adamw_step": torch.tensor(2.0), "ema_shadow": vec_state["ema_shadow"].cpu(),
                "ema_initialized": True},
        },
        "param_groups": [
            {"params": [0, 1], "lr": 1e-3, "betas": (0.9, 0.95), "eps": 1e-8,
             "weight_decay": WD, "momentum": 0.95, "muon_beta2": 0.95, "fraction": 0.5,
             "num_heads": None, "newton_schulz": "gram", "row_normalization": "normuon",
             "momentum_form": "heavy_ball", "dion_route": "matrix"},
            {"params": [2], "lr": 1e-3, "betas": (0.9, 0.95), "eps": 1e-8, "weight_decay": 0.0,
             "momentum": 0.95, "muon_beta2": 0.95, "fraction": 1.0, "num_heads": None,
             "newton_schulz": "gram", "row_normalization": "normuon",
             "momentum_form": "heavy_ball", "dion_route": "adamw"},
        ],
        "_ema_step_count": 2,
    }
    weights = [p.detach().clone() for p in mats + vecs]
    twins = []
    for state_dict in (layout, own):
        m2, v2 = params()
        with torch.no_grad():
            for p, w in zip(m2 + v2, weights):
                p.copy_(w)
        o2 = opt(m2, v2)
        o2.load_state_dict(state_dict)
        for step in range(2, 4):
            _grads(m2 + v2, 400 + step)
            o2.step()
        o2.ema.flush_pending_updates()
        twins.append((o2, m2 + v2))
    (a, pa), (b, pb) = twins
    _assert_same(a, pa, b, pb, "reference layout vs own checkpoint")
