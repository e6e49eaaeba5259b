"""The optimizer-integrated EMA on the GPU: schedule, GPU and CPU shadows,
checkpoints, weight swaps (behaviour of tests/test_ema.py:89-520 of the
reference, restated here).

Shadows are checked against a plain torch lerp of the live weights; where the
reference's tests demand exactness (swaps, checkpoints, a constant parameter)
the checks here are exact too.
"""

from __future__ import annotations

import copy

import pytest
import torch
from torch import nn

import dionw_amd as dionw
from dionw_amd import EMAConfig, EMADevice
from dionw_amd.ema import no_profile

pytestmark = pytest.mark.gpu


def _config(device: EMADevice, decay: float, *, every: int = 1, start: int = 0,
            final: float | None = None, ramp: int | None = None,
            gamma: float | None = None) -> EMAConfig:
    return EMAConfig(decay=decay, device=device, pin_memory=True, update_every_n_steps=every,
                     start_step=start, decay_final=final, decay_ramp_steps=ramp,
                     power_gamma=gamma)


def _weights(seed: int = 0) -> tuple[nn.Parameter, nn.Parameter]:
    """A 32 x 48 matrix (Dion route) and a 48-vector (AdamW route)."""
    g = torch.Generator().manual_seed(seed)
    return (nn.Parameter(torch.randn(32, 48, generator=g).cuda()),
            nn.Parameter(torch.randn(48, generator=g).cuda()))


def _dion(weights: tuple[nn.Parameter, nn.Parameter], ema: EMAConfig | None) -> dionw.Dion:
    matrix, vector = weights
    return dionw.Dion(
        [{"params": [vector], dionw.ROUTE_KEY: "adamw"},
         {"params": [matrix], dionw.ROUTE_KEY: "matrix", dionw.FRACTION_KEY: 0.5}],
        lr=1e-2, momentum=0.95, muon_beta2=0.95, betas=(0.9, 0.99), weight_decay=0.0,
        eps=1e-8, ema=ema)


def _train(weights, opt, steps: int = 1, seed: int = 100) -> None:
    g = torch.Generator().manual_seed(seed)
    for _ in range(steps):
        for w in weights:
            w.grad = torch.randn(w.shape, generator=g).cuda()
        opt.step()


def _shadow(opt, w) -> torch.Tensor:
    return opt.state[w]["ema_shadow"]


@pytest.mark.parametrize("device", list(EMADevice))
@pytest.mark.parametrize(("every", "start"), [(1, 0), (2, 0), (1, 3), (2, 3)])
def test_shadow_tracks_a_lerp_of_the_live_weights(device: EMADevice, every: int,
                                                  start: int) -> None:
    decay = 0.8
    weights = _weights()
    opt = _dion(weights, _config(device, decay, every=every, start=start))
    expected = None
    for step in range(1, 10):
        _train(weights, opt, seed=step)
        live = [w.detach().clone() for w in weights]
        if start:
            if step < start or (step - start) % every:
                continue
            first = step == start
        else:
            if step % every:
                continue
            first = expected is None
        expected = live if first else [e.lerp(x, 1 - decay**every)
                                       for e, x in zip(expected, live)]
    opt.ema.flush_pending_updates()
    for w, e in zip(weights, expected):
        s = _shadow(opt, w)
        assert s.device.type == ("cuda" if device is EMADevice.GPU else "cpu")
        torch.testing.assert_close(s.cuda(), e, rtol=1e-6, atol=1e-6)


def test_swapped_flag_follows_swap_and_restore() -> None:
    weights = _weights()
    opt = _dion(weights, _config(EMADevice.GPU, 0.9))
    assert not opt.ema_weights_swapped
    _train(weights, opt)
    assert opt.swap_ema_weights() and opt.ema_weights_swapped
    assert opt.restore_non_ema_weights() and not opt.ema_weights_swapped


@pytest.mark.parametrize("device", list(EMADevice))
def test_checkpoint_restores_shadows_and_step_count(device: EMADevice) -> None:
    weights = _weights()
    config = _config(device, 0.9)
    opt = _dion(weights, config)
    _train(weights, opt, steps=3)
    saved = opt.state_dict()
    again = _dion(weights, config)
    again.load_state_dict(saved)
    assert again.ema.step_count == 3
    for w in weights:
        assert _shadow(again, w).device == _shadow(opt, w).device
        assert torch.equal(_shadow(again, w), _shadow(opt, w))
    with pytest.raises(ValueError, match="without EMA"):
        _dion(weights, None).load_state_dict(saved)
    with pytest.raises(ValueError, match="non-negative"):
        again.ema.step_count = -1


@pytest.mark.parametrize("device", list(EMADevice))
def test_swap_puts_shadows_in_and_restore_takes_them_out(device: EMADevice) -> None:
    weights = _weights()
    opt = _dion(weights, _config(device, 0.5))
    assert not opt.swap_ema_weights()  # nothing to swap before the first update
    _train(weights, opt, steps=3)
    live = [w.detach().clone() for w in weights]
    assert opt.swap_ema_weights()
    for w in weights:
        assert torch.equal(w.detach(), _shadow(opt, w).cuda())
    assert opt.restore_non_ema_weights()
    for w, x in zip(weights, live):
        assert torch.equal(w.detach(), x)


def test_unchanging_parameter_keeps_an_exact_shadow() -> None:
    weights = _weights()
    opt = _dion(weights, _config(EMADevice.GPU, 0.999))
    for group in opt.param_groups:
        group["lr"] = 0.0
    _train(weights, opt, steps=20)
    for w in weights:
        assert torch.equal(_shadow(opt, w), w.detach())


def test_swap_guards_and_weights_without_gradients() -> None:
    matrix, vector = weights = _weights()
    opt = _dion(weights, _config(EMADevice.GPU, 0.5))
    g = torch.Generator().manual_seed(7)
    for _ in range(2):
        matrix.grad = torch.randn(matrix.shape, generator=g).cuda()
        opt.step()
    # The vector never had a gradient: its shadow is still its value.
    assert torch.equal(_shadow(opt, vector), vector.detach())
    assert opt.swap_ema_weights()
    with pytest.raises(RuntimeError, match="already swapped"):
        opt.swap_ema_weights()
    with pytest.raises(RuntimeError, match="swapped in"):
        opt.step()
    opt.restore_non_ema_weights()
    opt.step()


def test_swap_scoped_to_a_module() -> None:
    weights = _weights()
    opt = _dion(weights, _config(EMADevice.GPU, 0.5))
    _train(weights, opt)
    frozen = nn.Sequential(nn.Linear(4, 4).cuda().requires_grad_(False))
    with pytest.raises(ValueError, match="no optimizer-managed parameters"):
        opt.swap_ema_weights(frozen)
    with pytest.raises(ValueError, match="outside the optimizer"):
        opt.swap_ema_weights(nn.Linear(4, 4).cuda())


def test_cpu_staging_stays_out_of_the_checkpoint() -> None:
    weights = _weights()
    opt = _dion(weights, _config(EMADevice.CPU, 0.9))
    _train(weights, opt)
    for entry in opt.state_dict()["state"].values():
        assert "ema_shadow" in entry
        assert not {"ema_tmp_cpu", "ema_pending", "ema_event"} & set(entry)
    assert "ema_tmp_cpu" in opt.state[weights[0]]


@pytest.mark.parametrize(("saved_on", "loaded_on"), [(EMADevice.GPU, EMADevice.CPU),
                                                     (EMADevice.CPU, EMADevice.GPU)])
def test_checkpoint_moves_between_gpu_and_cpu_shadows(saved_on: EMADevice,
                                                      loaded_on: EMADevice) -> None:
    weights = _weights()
    first = _dion(weights, _config(saved_on, 0.8))
    _train(weights, first, steps=2)
    second = _dion(weights, _config(loaded_on, 0.8))
    # A deep copy stands for a save and load (torch's loader would keep tensors
    # that already sit on the right device shared between the two optimizers).
    second.load_state_dict(copy.deepcopy(first.state_dict()))
    for w in weights:
        assert _shadow(second, w).device.type == ("cuda" if loaded_on is EMADevice.GPU
                                                   else "cpu")
    g = torch.Generator().manual_seed(1)
    grads = [torch.randn(w.shape, generator=g).cuda() for w in weights]
    start = [w.detach().clone() for w in weights]
    for opt in (first, second):
        with torch.no_grad():
            for w, x in zip(weights, start):
                w.copy_(x)
        for w, gr in zip(weights, grads):
            w.grad = gr.clone()
        opt.step()
        # Both optimizers step the same weights: let a CPU snapshot finish
        # reading them before the other optimizer overwrites them.
        opt.ema.flush_pending_updates()
    for w in weights:
        assert torch.equal(_shadow(second, w).cuda(), _shadow(first, w).cuda())


def test_ramped_decay_drives_each_update() -> None:
    config = _config(EMADevice.GPU, 0.5, final=0.9, ramp=4)
    weights = _weights()
    opt = _dion(weights, config)
    expected = None
    for step in range(1, 7):
        _train(weights, opt, seed=step)
        live = [w.detach().clone() for w in weights]
        expected = live if expected is None else [
            e.lerp(x, 1 - config.decay_at_step(step)) for e, x in zip(expected, live)]
    for w, e in zip(weights, expected):
        torch.testing.assert_close(_shadow(opt, w), e, rtol=1e-6, atol=1e-6)


class _TorchAdamWWithEMA(dionw.IntegratedEMAOptimizer, torch.optim.AdamW):
    def __init__(self, params, ema: EMAConfig) -> None:
        super().__init__(params, lr=1e-2)
        self._init_integrated_ema(ema, no_profile)


@pytest.mark.parametrize("device", list(EMADevice))
def test_mixin_keeps_float32_shadows_of_bfloat16_weights(device: EMADevice) -> None:
    g = torch.Generator().manual_seed(0)
    w = nn.Parameter(torch.randn(64, 32, generator=g).to("cuda", torch.bfloat16))
    opt = _TorchAdamWWithEMA([w], _config(device, 0.7))
    expected = None
    for _ in range(4):
        w.grad = torch.randn(64, 32, generator=g).to("cuda", torch.bfloat16)
        opt.step()
        live = w.detach().float()
        expected = live if expected is None else expected.lerp(live, 1 - 0.7)
    opt.ema.flush_pending_updates()
    shadow = opt.state[w]["ema_shadow"]
    assert shadow.dtype == torch.float32
    torch.testing.assert_close(shadow.cuda(), expected, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("weight_decay", [0.0, 0.1])
@pytest.mark.parametrize("every", [1, 2])
def test_fused_ema_equals_the_separate_pass(weight_decay: float, every: int,
                                           monkeypatch: pytest.MonkeyPatch) -> None:
    """The shadow lerp taken inside the apply and AdamW passes is bit-identical
    to the separate EMA pass (same lerp arithmetic on the same new weights), on
    selected, decay-only and unchanged rows alike."""
    from dionw_amd import _lib
    from dionw_amd.ema.tracker import OptimizerIntegratedEMA

    def build():
        g = torch.Generator().manual_seed(3)
        weights = [nn.Parameter(torch.randn(64, 96, generator=g).cuda()),   # selected rows
                   nn.Parameter(torch.randn(32, 48, generator=g).cuda()),   # every row
                   nn.Parameter(torch.randn(96, generator=g).cuda())]       # AdamW
        opt = dionw.Dion(
            [{"params": [weights[0]], dionw.ROUTE_KEY: "matrix", dionw.FRACTION_KEY: 0.25},
             {"params": [weights[1]], dionw.ROUTE_KEY: "matrix", dionw.FRACTION_KEY: 1.0},
             {"params": [weights[2]], dionw.ROUTE_KEY: "adamw"}],
            lr=1e-2, weight_decay=weight_decay, ema=_config(EMADevice.GPU, 0.9, every=every))
        return weights, opt

    def run(fuse: bool):
        names: list[str] = []
        original = _lib.call

        def recording(name, *args):
            names.append(name)
            return original(name, *args)

        with monkeypatch.context() as m:
            m.setattr(_lib, "call", recording)
            if not fuse:
                m.setattr(OptimizerIntegratedEMA, "fusable_shadows", lambda self, params: None)
            weights, opt = build()
            g = torch.Generator().manual_seed(4)
            for _ in range(5):
                for w in weights:
                    w.grad = torch.randn(w.shape, generator=g).cuda()
                opt.step()
            opt.ema.flush_pending_updates()
        return weights, opt, names

    fused_w, fused_opt, fused_names = run(True)
    plain_w, plain_opt, plain_names = run(False)
    assert "dionw_apply_update_ema" in fused_names and "dionw_adamw_ema" in fused_names
    assert "dionw_apply_update_ema" not in plain_names
    for a, b in zip(fused_w, plain_w):
        assert torch.equal(a.detach(), b.detach())
        assert torch.equal(_shadow(fused_opt, a), _shadow(plain_opt, b))


@pytest.mark.parametrize("every", [1, 2])
def test_cpu_ema_copies_started_after_each_pass_equal_end_of_step_copies(
        every: int, monkeypatch: pytest.MonkeyPatch) -> None:
    """CPU EMA: the host copies of each run's (and the AdamW group's) new
    weights start right after the pass that wrote them; the shadows equal those
    of copies staged after the whole step, bit for bit."""
    from dionw_amd.ema.tracker import OptimizerIntegratedEMA

    def run(early: bool):
        with monkeypatch.context() as m:
            if not early:
                m.setattr(OptimizerIntegratedEMA, "stage_written", lambda self, params: None)
            g = torch.Generator().manual_seed(5)
            weights = [nn.Parameter(torch.randn(64, 96, generator=g).cuda()),
                       nn.Parameter(torch.randn(64, 96, generator=g).cuda()),
                       nn.Parameter(torch.randn(96, generator=g).cuda())]
            opt = dionw.Dion(
                [{"params": weights[:2], dionw.ROUTE_KEY: "matrix", dionw.FRACTION_KEY: 0.5},
                 {"params": weights[2:], dionw.ROUTE_KEY: "adamw"}],
                lr=1e-2, weight_decay=0.1, ema=_config(EMADevice.CPU, 0.9, every=every))
            for _ in range(5):
                for w in weights:
                    w.grad = torch.randn(w.shape, generator=g).cuda()
                opt.step()
            opt.ema.flush_pending_updates()
            return [_shadow(opt, w).clone() for w in weights], [w.detach().cpu() for w in weights]

    early_shadows, early_weights = run(True)
    late_shadows, late_weights = run(False)
    for a, b in zip(early_weights, late_weights):
        assert torch.equal(a, b)
    for a, b in zip(early_shadows, late_shadows):
        assert a.device.type == "cpu" and torch.equal(a, b)
    assert not torch.equal(early_shadows[0], early_weights[0])  # a real lerp, not a copy


@pytest.mark.parametrize(("weight_decay", "fraction", "start"),
                         [(0.1, 0.5, 0), (0.0, 0.5, 0), (0.0, 1.0, 0), (0.1, 0.25, 3)])
def test_cpu_ema_snapshots_written_by_the_apply_pass_equal_copied_ones(
        weight_decay: float, fraction: float, start: int,
        monkeypatch: pytest.MonkeyPatch) -> None:
    """CPU EMA: the matrix apply pass writes each parameter's host snapshot
    itself (every row, also rows neither selected nor decayed), and the shadows
    equal those of snapshots copied on the copy stream, bit for bit, through a
    restart from the live weights (start_step) and lerps."""
    from dionw_amd import _lib

    original = _lib.call

    def run(fuse: bool):
        names: list[str] = []

        def recording(name, *args):
            names.append(name)
            return original(name, *args)

        monkeypatch.setattr(_lib, "call", recording)
        g = torch.Generator().manual_seed(9)
        weights = [nn.Parameter(torch.randn(128, 96, generator=g).cuda()),
                   nn.Parameter(torch.randn(128, 96, generator=g).cuda()),
                   nn.Parameter(torch.randn(96, 130, generator=g).cuda()),
                   nn.Parameter(torch.randn(96, generator=g).cuda())]
        opt = dionw.Dion(
            [{"params": weights[:3], dionw.ROUTE_KEY: "matrix", dionw.FRACTION_KEY: fraction},
             {"params": weights[3:], dionw.ROUTE_KEY: "adamw"}],
            lr=1e-2, weight_decay=weight_decay, ema=_config(EMADevice.CPU, 0.9, start=start))
        opt.ema.fuse_host_copies = fuse
        for _ in range(6):
            for w in weights:
                w.grad = torch.randn(w.shape, generator=g).cuda()
            opt.step()
        opt.ema.flush_pending_updates()
        monkeypatch.setattr(_lib, "call", original)
        return ([_shadow(opt, w).clone() for w in weights], [w.detach().cpu() for w in weights],
                names)

    fused_shadows, fused_weights, fused_names = run(True)
    copied_shadows, copied_weights, copied_names = run(False)
    assert "dionw_apply_update_stage" in fused_names
    assert "dionw_apply_update_stage" not in copied_names
    for a, b in zip(fused_weights, copied_weights):
        assert torch.equal(a, b)
    for a, b in zip(fused_shadows, copied_shadows):
        assert a.device.type == "cpu" and torch.equal(a, b)
    assert not torch.equal(fused_shadows[0], fused_weights[0])  # a real lerp, not a copy


def test_apply_stage_writes_every_row_to_pinned_host_memory() -> None:
    """dionw_apply_update_stage through the C ABI: with row selection and no
    weight decay, the host buffers receive every row of the new weights (the
    unselected rows unchanged), and the device update equals dionw_apply_update's."""
    from dionw_amd import _lib

    g = torch.Generator().manual_seed(3)
    blocks_per, rows, cols, k, count = 2, 64, 72, 16, 3
    start = [torch.randn(blocks_per * rows, cols, generator=g) for _ in range(count)]
    orth = (torch.randn(count * blocks_per, k, cols, generator=g) * 0.1).to(torch.bfloat16)
    idx = torch.stack([torch.randperm(rows, generator=g)[:k].sort().values
                       for _ in range(count * blocks_per)]).to(torch.int32)
    slot = torch.full((count * blocks_per, rows), -1, dtype=torch.int32)
    for b in range(count * blocks_per):
        slot[b, idx[b].long()] = torch.arange(k, dtype=torch.int32)
    dev = [t.cuda() for t in (orth, idx, slot)]
    plain = [t.clone().cuda() for t in start]
    staged_w = [t.clone().cuda() for t in start]
    # The last buffer is a view that starts inside a larger pinned allocation:
    # the device address the library looks up must keep its offset.
    host = [torch.full_like(t, float("nan")).pin_memory() for t in start[:-1]]
    pool = torch.full((2 * start[-1].numel() + 4,), float("nan")).pin_memory()
    host.append(pool[start[-1].numel() + 4:].view(start[-1].shape))
    common = (count, blocks_per, rows, cols, k, dev[0].data_ptr(), dev[1].data_ptr(),
              dev[2].data_ptr(), None, None, 0.5, 1.0, 0)
    stream = _lib.stream_handle()
    _lib.call("dionw_apply_update", _lib.ptr_array(plain), *common, stream)
    _lib.call("dionw_apply_update_stage", _lib.ptr_array(staged_w), _lib.ptr_array(host),
              *common, stream)
    torch.cuda.synchronize()
    for p, s, h, w0 in zip(plain, staged_w, host, start):
        assert torch.equal(p, s)
        assert torch.equal(h, s.cpu())
        assert not torch.equal(h, w0)
    assert bool(pool[: start[-1].numel() + 4].isnan().all())  # nothing written before the view


def test_apply_stage_rejects_memory_that_is_not_pinned_host_memory() -> None:
    """Device memory or pageable host memory as a staging buffer is refused on
    the host, before any launch, and leaves no HIP error behind."""
    from dionw_amd import _lib

    w = [torch.zeros(8, 16, device="cuda")]
    orth = torch.zeros(1, 8, 16, dtype=torch.bfloat16, device="cuda")
    common = (1, 1, 8, 16, 8, orth.data_ptr(), None, None, None, None, 0.5, 1.0, 0)
    stream = _lib.stream_handle()
    for bad in (torch.zeros(8, 16, device="cuda"), torch.zeros(8, 16)):
        with pytest.raises(ValueError, match="pinned host memory"):
            _lib.call("dionw_apply_update_stage", _lib.ptr_array(w), _lib.ptr_array([bad]),
                      *common, stream)
    torch.cuda.synchronize()
    assert torch.equal(w[0], torch.zeros_like(w[0]))
    torch.zeros(4, device="cuda").add_(1)  # the runtime is still usable
    torch.cuda.synchronize()
