"""Host logic of the optimizer and the EMA that needs no GPU.

Run splitting (reference tests/test_optimizer.py:688-730), the EMA cadence
(tests/test_ema.py:141-205), the CPU EMA worker's error path
(ema/_cpu_job.py:36-43, 104-137), swap planning (tests/test_ema.py:320-362),
group validation messages (tests/test_optimizer.py:455-480, 740-798) and the
scratch-buffer keying.
"""

from __future__ import annotations

import pytest
import torch
from torch import nn

from dionw_amd import _workspace
from dionw_amd import optimizer as opt_module
from dionw_amd._buckets import Bucket
from dionw_amd._groups import GroupSpec, check_decays, check_parameter, matrix_blocks
from dionw_amd.ema import EMAConfig
from dionw_amd.ema._host_worker import HostEmaWorker, HostSnapshot
from dionw_amd.ema._keys import EMA_INITIALIZED, EMA_PENDING
from dionw_amd.ema._swap import WeightSwap, swap_plan
from dionw_amd.ema.tracker import cadence_at


def _bucket(block_counts: list[int], grads: list[bool], rows: int = 32, cols: int = 48,
            selected: int = 32) -> Bucket:
    params = []
    for count, has_grad in zip(block_counts, grads):
        p = nn.Parameter(torch.zeros(count * rows, cols))
        p.grad = torch.zeros_like(p) if has_grad else None
        params.append(p)
    offsets = [0]
    for count in block_counts:
        offsets.append(offsets[-1] + count)
    n = offsets[-1]
    return Bucket(0, lambda x, e: x, params, offsets, rows, cols, selected,
                  torch.zeros(n, rows, cols), torch.zeros(n, rows, 1))


def test_runs_split_at_missing_gradients_and_the_cap(monkeypatch) -> None:
    bucket = _bucket([1, 1, 1, 1, 1], [True, True, False, True, True])
    assert list(opt_module._runs(bucket)) == [[0, 1], [3, 4]]
    monkeypatch.setattr(opt_module, "MAX_RUN_ELEMENTS", 2 * 32 * 48)
    four = _bucket([1, 1, 1, 1], [True] * 4)
    assert list(opt_module._runs(four)) == [[0, 1], [2, 3]]
    # a parameter larger than the cap runs alone; selected rows count, not rows
    big = _bucket([3, 1, 1], [True] * 3, selected=8)
    monkeypatch.setattr(opt_module, "MAX_RUN_ELEMENTS", 2 * 8 * 48)
    assert list(opt_module._runs(big)) == [[0], [1, 2]]
    assert list(opt_module._runs(_bucket([1, 1], [False, False]))) == []


def test_bucket_block_ranges_and_views() -> None:
    bucket = _bucket([2, 1, 3], [True] * 3)
    assert bucket.blocks_per_param == 2
    assert bucket.param_blocks(2) == slice(3, 6)
    assert bucket.run_blocks([1, 2]) == slice(2, 6)
    state: dict = {bucket.params[1]: {"momentum": torch.ones(32, 48)}}
    state.setdefault(bucket.params[0], {})
    state.setdefault(bucket.params[2], {})
    bucket.adopt(state)
    assert torch.equal(bucket.momentum[2], torch.ones(32, 48))  # an existing entry is copied in
    assert state[bucket.params[2]]["momentum"].untyped_storage().data_ptr() == \
        bucket.momentum.untyped_storage().data_ptr()
    assert state[bucket.params[2]]["variance"].shape == (96, 1)


def test_matrix_blocks() -> None:
    assert matrix_blocks(torch.zeros(64, 3, 3, 8), None) == (1, 64, 72)
    assert matrix_blocks(torch.zeros(96, 16), 3) == (3, 32, 16)
    with pytest.raises(ValueError, match="does not divide"):
        matrix_blocks(torch.zeros(30, 16), 4)


def test_ema_cadence_table() -> None:
    every2 = EMAConfig(decay=0.9, update_every_n_steps=2)
    table = [cadence_at(every2, n) for n in range(1, 6)]
    assert [c.update for c in table] == [False, True, False, True, False]
    assert table[1].decay == pytest.approx(0.81) and not table[1].from_live
    delayed = EMAConfig(decay=0.9, update_every_n_steps=2, start_step=3)
    table = [cadence_at(delayed, n) for n in range(1, 8)]
    assert [c.update for c in table] == [False, False, True, False, True, False, True]
    assert table[2].from_live and table[2].decay is None
    ramp = EMAConfig(decay=0.9, decay_final=0.99, decay_ramp_steps=10)
    assert cadence_at(ramp, 5).decay == pytest.approx(0.945)
    power = EMAConfig(decay=0.999, power_gamma=1.0)
    assert cadence_at(power, 2).decay == pytest.approx(0.25)


def test_host_worker_rejects_device_buffers_and_reraises_failures() -> None:
    entry = {EMA_INITIALIZED: True, EMA_PENDING: True}
    with pytest.raises(ValueError, match="must live on the CPU"):
        HostSnapshot(entry, None, torch.zeros(4), torch.zeros(4, device="meta"))
    worker = HostEmaWorker()
    bad = HostSnapshot(entry, None, torch.zeros(4), torch.zeros(5))  # shapes disagree
    worker.submit([bad], decay=0.9)
    with pytest.raises(RuntimeError, match="CPU EMA update failed"):
        worker.wait()
    worker.wait()  # the failure is reported once
    shadow, staged = torch.zeros(4), torch.full((4,), 2.0)
    good = {EMA_INITIALIZED: False, EMA_PENDING: True}
    worker.submit([HostSnapshot(good, None, shadow, staged)], decay=0.9)
    worker.wait()
    assert torch.equal(shadow, staged) and good[EMA_INITIALIZED] and not good[EMA_PENDING]
    worker.submit([HostSnapshot(good, None, shadow, torch.zeros(4, dtype=torch.bfloat16))],
                  decay=0.5)
    worker.wait()
    assert torch.equal(shadow, torch.ones(4))  # lerp through the float32 scratch


def test_swap_plan_and_weight_swap() -> None:
    a, b = nn.Parameter(torch.ones(3)), nn.Parameter(torch.ones(2))
    state = {a: {"ema_shadow": torch.zeros(3)}, b: {"ema_shadow": torch.full((2,), 5.0)}}
    pairs = swap_plan(None, [a, b], state, "Dion")
    swap = WeightSwap()
    assert swap.apply(pairs) and swap.active
    assert torch.equal(a.data, torch.zeros(3))
    with pytest.raises(RuntimeError, match="already swapped"):
        swap.apply(pairs)
    swap.undo()
    assert not swap.active and torch.equal(a.data, torch.ones(3))
    assert swap_plan(None, [a], {}, "Dion") == []  # before the first update
    with pytest.raises(RuntimeError, match="mix live and EMA weights"):
        swap_plan(None, [a, b], {a: state[a]}, "Dion")
    with pytest.raises(ValueError, match="outside the optimizer"):
        swap_plan(nn.Linear(2, 2), [a, b], state, "Dion")
    with pytest.raises(ValueError, match="no optimizer-managed parameters"):
        swap_plan(nn.Linear(2, 2).requires_grad_(False), [a, b], state, "Dion")
    with pytest.raises(ValueError, match="No parameters"):
        swap_plan(None, [], state, "Dion")


def _group(**extra) -> dict:
    base = {"params": [torch.zeros(8, 8)], "lr": 1e-3, "weight_decay": 0.0, "fraction": 1.0,
            "num_heads": None, "newton_schulz": "gram", "row_normalization": "normuon",
            "momentum_form": "heavy_ball", "dion_route": "matrix"}
    base.update(extra)
    return base


def test_group_spec_messages() -> None:
    spec = GroupSpec.of(_group(fraction=0.5))
    assert spec.fraction == 0.5 and spec.num_heads is None
    no_route = _group()
    del no_route["dion_route"]
    with pytest.raises(TypeError, match=r"dionw\.param_groups"):
        GroupSpec.of(no_route)
    with pytest.raises(ValueError, match="fraction"):
        GroupSpec.of(_group(fraction=1.5))
    with pytest.raises(ValueError, match="Nesterov momentum needs every row"):
        GroupSpec.of(_group(fraction=0.5, momentum_form="nesterov"))
    with pytest.raises(ValueError, match="route it to AdamW"):
        GroupSpec.of(_group(params=[torch.zeros(8)]))
    with pytest.raises(ValueError, match="does not divide"):
        GroupSpec.of(_group(params=[torch.zeros(30, 16)], num_heads=4))
    with pytest.raises(ValueError, match="lr and weight_decay"):
        GroupSpec.of(_group(lr=-1.0))
    with pytest.raises(ValueError, match="'row_normalization'|is not a valid"):
        GroupSpec.of(_group(row_normalization="bogus"))
    with pytest.raises(ValueError, match="momentum"):
        check_decays(lr=1.0, weight_decay=0.0, eps=1e-8, decays={"momentum": 1.0})
    with pytest.raises(ValueError, match="lr and weight_decay"):
        check_decays(lr=1.0, weight_decay=0.0, eps=0.0, decays={})
    with pytest.raises(ValueError, match="CUDA"):
        check_parameter(torch.zeros(2, 2))


def test_workspace_is_keyed_by_device_and_stream() -> None:
    cpu = torch.device("cpu")
    _workspace.release(cpu)
    a = _workspace.buffer(cpu, "t", (4,), torch.float32, stream=1)
    b = _workspace.buffer(cpu, "t", (4,), torch.float32, stream=2)
    assert a.data_ptr() != b.data_ptr()
    assert _workspace.buffer(cpu, "t", (2,), torch.float32, stream=1).data_ptr() == a.data_ptr()
    grown = _workspace.buffer(cpu, "t", (1000,), torch.float32, stream=1)
    assert grown.numel() == 1000 and _workspace.held_bytes(cpu) >= 4000
    import dionw_amd
    dionw_amd.release_workspace(cpu)  # the public name of the same release
    assert _workspace.held_bytes(cpu) == 0


def test_workspace_share_aliases_only_missing_names() -> None:
    """A capture stream sees the eager stream's buffers (same storage), keeps
    the ones it already has, and a shared buffer is counted once."""
    cpu = torch.device("cpu")
    _workspace.release(cpu)
    a = _workspace.buffer(cpu, "a", (64,), torch.float32, stream=1)
    _workspace.buffer(cpu, "b", (64,), torch.float32, stream=1)
    own = _workspace.buffer(cpu, "b", (8,), torch.float32, stream=2)
    before = _workspace.held_bytes(cpu)
    _workspace.share(cpu, 1, 2)
    assert _workspace.buffer(cpu, "a", (64,), torch.float32, stream=2).data_ptr() == a.data_ptr()
    assert _workspace.buffer(cpu, "b", (8,), torch.float32, stream=2).data_ptr() == own.data_ptr()
    assert _workspace.held_bytes(cpu) == before
    assert len(_workspace.tensors(cpu)) == 4  # (1, a), (1, b), (2, b), (2, a)
    _workspace.release(cpu)
    assert _workspace.tensors(cpu) == []


def test_step_graph_records_only_a_dion() -> None:
    from dionw_amd import StepGraph
    param = nn.Parameter(torch.zeros(4, 4))
    with pytest.raises(TypeError, match="Dion"):
        StepGraph(torch.optim.SGD([param], lr=0.1))


def test_workspace_release_resolves_the_current_gpu(monkeypatch) -> None:
    """``cuda`` names the current GPU: buffers kept under ``cuda:0`` are counted
    and released through ``cuda`` as well (an index-less device must not match
    nothing). A CPU tensor stands in for the GPU buffer; nothing is launched."""
    monkeypatch.setattr(torch.cuda, "current_device", lambda: 0)
    assert _workspace._resolved("cuda") == torch.device("cuda", 0)
    assert _workspace._resolved("cuda:1") == torch.device("cuda", 1)
    assert _workspace._resolved("cpu") == torch.device("cpu")
    key = (torch.device("cuda", 0), 0, "stand_in")
    monkeypatch.setitem(_workspace._BUFFERS, key, torch.zeros(512, dtype=torch.uint8))
    assert _workspace.held_bytes("cuda") >= 512
    assert _workspace.held_bytes(torch.device("cuda", 1)) == 0
    import dionw_amd
    dionw_amd.release_workspace("cuda")
    assert key not in _workspace._BUFFERS and _workspace.held_bytes("cuda") == 0


def test_step_stages_run_in_named_regions_in_step_order(monkeypatch) -> None:
    """``profile_region`` marks every stage of a step, in step order: each run's
    momentum passes, then the queued Newton-Schulz products, each run's finish
    (NorMuon statistics and the weight update), then the AdamW groups. The
    library calls are recorded instead of executed (CPU tensors stand in for
    GPU ones, nothing is launched), so the test also pins which entry points
    each stage issues."""
    import contextlib

    from dionw_amd import _groups, _lib, _matrix_step

    events: list[tuple[str, str]] = []
    depth = []

    @contextlib.contextmanager
    def region(name: str):
        assert not depth, f"region {name} opened inside {depth[-1]}"
        depth.append(name)
        events.append(("region", name))
        try:
            yield
        finally:
            depth.pop()

    def record(name: str, *args) -> None:
        events.append(("call", name))

    monkeypatch.setattr(_lib, "call", record)
    monkeypatch.setattr(_lib, "stream_handle", lambda device=None: 0)
    monkeypatch.setattr(_groups, "check_parameter", lambda param: None)
    monkeypatch.setattr(opt_module, "check_parameter", lambda param: None)
    # One stream for the flush (a second one would need a GPU).
    monkeypatch.setattr(_matrix_step, "_lanes", lambda calls, grouped: [list(range(len(calls)))])
    g = torch.Generator().manual_seed(0)
    wide = [nn.Parameter(torch.randn(64, 256, generator=g)) for _ in range(2)]
    wider = nn.Parameter(torch.randn(64, 512, generator=g))
    bias = nn.Parameter(torch.zeros(64))
    opt = opt_module.Dion(
        [{"params": [*wide, wider], "dion_route": "matrix", "fraction": 0.25},
         {"params": [bias], "dion_route": "adamw"}],
        lr=1e-3, profile_region=region)
    for p in (*wide, wider, bias):
        p.grad = torch.randn(p.shape, generator=g)
    opt.step()
    regions = [name for kind, name in events if kind == "region"]
    # Two buckets (64x256 and 64x512 blocks): momentum passes per run, then
    # the queue's products (grouped or one call per run) and each run's finish.
    assert regions[:2] == ["dion_momentum", "dion_momentum"]
    assert regions[-1] == "adamw"
    middle = regions[2:-1]
    assert middle.count("dion_finish") == 2 and "dion_orthogonalize" in middle
    assert middle.index("dion_orthogonalize") < middle.index("dion_finish")
    stage = None
    issued: dict[str, set[str]] = {}
    for kind, name in events:
        if kind == "region":
            stage = name
        else:
            assert stage is not None, f"{name} issued outside every region"
            issued.setdefault(stage, set()).add(name)
    assert issued["dion_momentum"] == {"dionw_accumulate_scores", "dionw_select_rows",
                                       "dionw_prepare_ns_input"}
    assert issued["dion_orthogonalize"] <= {"dionw_newton_schulz", "dionw_newton_schulz_group"}
    assert issued["dion_finish"] == {"dionw_normuon_stats", "dionw_apply_update"}
    assert issued["adamw"] == {"dionw_increment_steps", "dionw_adamw"}


def test_queue_keeps_at_most_its_byte_cap(monkeypatch) -> None:
    """The queue's per-position scratch is reused across flushes and steps, and
    dropped before growing one position would take the total past the byte cap:
    what it keeps stays within the cap, or one run's buffers when a run alone is
    larger. CPU buffers stand in for the GPU's; the products are not launched."""
    from dionw_amd import _matrix_step
    from dionw_amd._matrix_step import RunQueue

    cpu = torch.device("cpu")
    monkeypatch.setattr(_matrix_step, "QUEUE_BYTES", 10_000)
    monkeypatch.setattr(_matrix_step, "group_launches", lambda calls: len(calls))
    monkeypatch.setattr(_matrix_step, "run_newton_schulz_call", lambda call, stream: None)
    monkeypatch.setattr(_matrix_step, "run_newton_schulz_group", lambda calls, stream: None)
    monkeypatch.setattr(_matrix_step, "_lanes", lambda calls, grouped: [list(range(len(calls)))])
    _workspace.release(cpu)
    queue = RunQueue()
    kept = lambda: _workspace.named_bytes(cpu, 0, lambda name: "#" in name)  # noqa: E731

    def run(nbytes: int) -> str:
        own = queue.slot(nbytes, 0, cpu)
        _workspace.buffer(cpu, "ns_out" + own, (nbytes,), torch.uint8, stream=0)
        queue.add(object(), lambda: None, nbytes, 0, cpu)
        return own

    assert [run(3000) for _ in range(3)] == ["#0", "#1", "#2"]
    queue.flush()
    assert kept() <= 10_000
    # Growing position 0 to 9000 next to 6000 kept elsewhere would pass the cap:
    # every position's buffers are dropped first.
    assert run(9000) == "#0" and kept() <= 10_000
    assert run(3000) == "#0"  # does not fit beside the 9000 queued: flushed, reused
    queue.flush()
    assert kept() <= 10_000
    # A run larger than the cap alone: kept, nothing else beside it.
    assert run(25_000) == "#0" and 25_000 <= kept() < 25_000 + 256  # 256-byte alignment
    queue.flush()
    assert run(100) == "#0" and kept() < 25_000 + 256
    queue.flush()
    _workspace.release(cpu)
