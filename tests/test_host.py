"""Host-side logic and the C ABI's presence (no GPU needed).

Restates the reference's routing table (tests/test_routing.py:38-190), config
validation, EMA schedule known answers (tests/test_ema.py:141-205) and the
structural checks of load_state_dict (tests/test_optimizer.py:776-798).
"""

from __future__ import annotations

import ctypes
import json
import math
import re
from pathlib import Path

import pytest
import torch
from torch import nn

import dionw_amd
from dionw_amd import EMAConfig, Route, RouteKind, RouteReason, param_groups
from dionw_amd import _lib
from dionw_amd._groups import refuse_structural_change

HEADER = Path(__file__).resolve().parents[1] / "include" / "dionw_hip.h"


def test_library_exports_every_declared_symbol() -> None:
    declared = set(re.findall(r"^\w[\w\s\*]*?\b(dionw_\w+)\s*\(", HEADER.read_text(), re.M))
    assert declared, "no declarations parsed"
    assert declared == set(_lib.SIGNATURES), "ctypes table and header disagree"
    lib = ctypes.CDLL(str(_lib.library_path()))
    for name in declared:
        assert hasattr(lib, name), f"{name} not exported"
    assert _lib.library().dionw_abi_version() == 2


@pytest.mark.parametrize(("kind", "table"), [(0, "gram"), (1, "polar_express"), (2, "keller"),
                                             (3, "polar_express"), (4, "keller")])
def test_library_coefficient_tables_equal_the_reference_literals(kind: int, table: str) -> None:
    """The five (a, b, c) rows each library kind runs against the reference's
    literal tables (tests/golden/coefficients.json); the Gram rows with the
    safety factor folded in as _gram.py:32-35 does."""
    fx = json.loads((Path(__file__).resolve().parent / "golden" / "coefficients.json").read_text())
    if table == "gram":
        s = fx["gram_safety"]
        want = [(a / s, b / s**3, c / s**5) for a, b, c in fx["gram_unmodified"]]
    else:
        want = [tuple(r) for r in fx[table]]
    out = (ctypes.c_double * 15)()
    _lib.call("dionw_ns_coefficients", kind, out)
    got = [tuple(out[3 * i:3 * i + 3]) for i in range(5)]
    for row_got, row_want in zip(got, want, strict=True):
        for g, w in zip(row_got, row_want):
            assert math.isclose(g, w, rel_tol=1e-15), (kind, got, want)
    with pytest.raises(ValueError, match="unknown kind"):
        _lib.call("dionw_ns_coefficients", 5, out)


def test_gemm_nt_rejects_mismatched_operands() -> None:
    """gemm_nt checks shapes, batches, dtypes and devices on the host before any
    launch (a mismatched operand would otherwise be read or written out of
    bounds)."""
    from dionw_amd._kernels import gemm_nt

    a = torch.zeros(2, 64, 32, dtype=torch.float16)
    with pytest.raises(ValueError, match="does not match"):
        gemm_nt(a, torch.zeros(2, 64, 48, dtype=torch.float16))      # k differs
    with pytest.raises(ValueError, match="does not match"):
        gemm_nt(a, torch.zeros(3, 64, 32, dtype=torch.float16))      # batch differs
    with pytest.raises(ValueError, match="both be 2-D or 3-D"):
        gemm_nt(a, torch.zeros(64, 32, dtype=torch.float16))
    b = torch.zeros(2, 40, 32, dtype=torch.float16)
    with pytest.raises(ValueError, match="out must be"):
        gemm_nt(a, b, out=torch.zeros(2, 64, 41, dtype=torch.float16))
    with pytest.raises(ValueError, match="out_t must be"):
        gemm_nt(a, b, out_t=torch.zeros(2, 64, 40, dtype=torch.float16))
    with pytest.raises(ValueError, match="d must be"):
        gemm_nt(a, b, d=torch.zeros(2, 40, 64, dtype=torch.float16), beta=1.0)
    with pytest.raises(ValueError, match="share a's dtype"):
        gemm_nt(a, b.to(torch.bfloat16))
    with pytest.raises(ValueError, match="unit column stride"):
        gemm_nt(a, torch.zeros(2, 32, 40, dtype=torch.float16).mT)
    with pytest.raises(ValueError, match="unsupported dtype"):
        gemm_nt(a.double(), b.double())
    with pytest.raises(ValueError, match="symmetric"):
        gemm_nt(a, b, symmetric=True)


def test_momentum_seams_take_any_float_gradient_and_reject_others() -> None:
    """accumulate_row_l1 / accumulate_copy_decay accept float16, bfloat16 and
    float32 gradients like the reference's kernels (_momentum_kernels.py:89-133);
    integer gradients and mismatched sizes are rejected before any launch."""
    from dionw_amd._kernels import _check

    m = torch.zeros(4, 8)
    for dtype in (torch.float16, torch.bfloat16, torch.float32):
        g = torch.randn(4, 8).to(dtype)
        got = _check(g, m)
        assert got.dtype == torch.float32 and torch.equal(got, g.float())
    with pytest.raises(ValueError, match="float gradient"):
        _check(torch.zeros(4, 8, dtype=torch.int32), m)
    with pytest.raises(ValueError, match="float32 momentum"):
        _check(torch.zeros(4, 9), m)
    with pytest.raises(ValueError, match="contiguous"):
        _check(torch.zeros(8, 4).mT, m)


def test_grouped_newton_schulz_rejects_overlapping_workspaces() -> None:
    """Runs of one grouped call execute together, so their workspaces must be
    disjoint; the host rejects the call before any launch (the fake device
    addresses below are never dereferenced)."""
    n = 2
    need = int(_lib.library().dionw_newton_schulz_workspace(0, 1, 64, 128))
    base = 1 << 40

    def arr(ctype, *values):
        return (ctype * n)(*values)

    i32, i64, ptr = ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p
    args = [arr(i32, 0, 0), arr(i64, 1, 1), arr(i64, 64, 64), arr(i64, 128, 128),
            arr(ptr, base, base + 2**30), arr(ptr, base + 2**31, base + 2**32),
            arr(i64, 64, 64), arr(i64, 128, 128), arr(ptr, base + 2**33, base + 2**34),
            arr(i32, 0, 0), arr(i64, 128, 128), arr(i64, 64 * 128, 64 * 128)]
    with pytest.raises(ValueError, match="overlap"):
        _lib.call("dionw_newton_schulz_group", n, *args,
                  arr(ptr, base + 2**35, base + 2**35 + need // 2),
                  arr(ctypes.c_size_t, need, need), None)
    with pytest.raises(ValueError, match="bad count"):
        _lib.call("dionw_newton_schulz_group", -1, *args, arr(ptr, base, base),
                  arr(ctypes.c_size_t, 0, 0), None)


def test_normuon_stats_rejects_negative_block_counts() -> None:
    """A negative block count is rejected by both NorMuon statistics entry
    points before any launch or device lookup (the fake addresses are never
    dereferenced; a wrapped count would otherwise size a huge grid)."""
    fake = 1 << 40
    args = (fake, -1, 4, 8, 16, fake, fake, 0.95, -0.01, fake)
    with pytest.raises(ValueError, match="bad sizes"):
        _lib.call("dionw_normuon_stats", *args, fake, fake, None)
    with pytest.raises(ValueError, match="bad sizes"):
        _lib.call("dionw_normuon_stats_noalloc", *args, fake, None)
    with pytest.raises(ValueError, match="exceed one launch"):
        _lib.call("dionw_normuon_stats", fake, 1 << 31, 4, 8, 16, fake, fake, 0.95, -0.01, fake,
                  fake, fake, None)


def test_prepared_orientations() -> None:
    """The iterate is the wide orientation; its transpose is prepared only when
    the short side, rounded up to 8, is not a multiple of 32."""
    from dionw_amd.newton_schulz import prepared_orientations

    assert prepared_orientations(256, 1024) == (True, False)
    assert prepared_orientations(1024, 256) == (False, True)  # tall: iterates on the transpose
    assert prepared_orientations(128, 128) == (True, False)
    assert prepared_orientations(30, 300) == (True, False)    # round8(30) = 32
    assert prepared_orientations(300, 30) == (False, True)
    assert prepared_orientations(100, 200) == (True, True)    # round8(100) = 104
    assert prepared_orientations(200, 100) == (True, True)
    assert prepared_orientations(72, 72) == (True, True)


def test_padded_short_side_never_exceeds_the_long_side() -> None:
    """Padding a short side that is an odd multiple of 32 to a multiple of 64
    keeps the iteration's orientation: over square, near-square and ragged
    shapes, the padded side the iteration treats as short (the unpadded short
    side) is never longer than the other, both are rounded up to 8 at least, and
    the library plans the call (launch count from shapes alone, no GPU)."""
    from dionw_amd.newton_schulz import padded_sides

    sides = [8, 30, 100, 256, 264, 280, 288, 296, 312, 320, 352, 384, 416, 1408, 1440, 1472,
             2048, 3584]
    for rows in sides:
        for cols in sides + [rows + d for d in (1, 8, 31, 32, 33)]:
            for a, b in ((rows, cols), (cols, rows)):
                p_pad, j_pad = padded_sides(a, b)
                assert p_pad >= a and j_pad >= b and p_pad % 8 == 0 and j_pad % 8 == 0
                r, c = (j_pad, p_pad) if a > b else (p_pad, j_pad)
                assert r <= c, f"[{a}, {b}] padded to ({p_pad}, {j_pad})"
                i64 = ctypes.c_int64
                planned = _lib.library().dionw_newton_schulz_group_launches(
                    1, (ctypes.c_int32 * 1)(0), (i64 * 1)(1), (i64 * 1)(r), (i64 * 1)(c),
                    (i64 * 1)(min(a, b)), (i64 * 1)(max(a, b)))
                assert planned > 0, (a, b)
    assert padded_sides(288, 288) == (288, 288)
    assert padded_sides(288, 296) == (288, 296)
    assert padded_sides(1440, 1440) == (1440, 1440)
    assert padded_sides(352, 2048) == (384, 2048)   # MoE gate/up iterate: padded
    assert padded_sides(2048, 352) == (2048, 384)   # its tall twin


def test_newton_schulz_needs_the_transpose_it_reads() -> None:
    """Where r is not a multiple of 32 the products read X^T: a NULL xt is
    rejected before any launch (fake addresses, never dereferenced); the host
    wrapper rejects a missing input the same way."""
    from dionw_amd.newton_schulz import NewtonSchulz, newton_schulz_call, newton_schulz_fn

    need = int(_lib.library().dionw_newton_schulz_workspace(0, 1, 104, 200))
    fake = 1 << 40
    with pytest.raises(ValueError, match="null pointer"):
        _lib.call("dionw_newton_schulz", 0, 1, 104, 200, fake, None, 100, 200, fake, 0, 200,
                  100 * 200, fake + 2**30, need, None)
    ortho = newton_schulz_fn(NewtonSchulz.GRAM)
    out = torch.empty(1, 100, 200, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="prepared"):
        newton_schulz_call(ortho, 1, 100, 200, torch.empty(1, 104, 200, dtype=torch.half), None,
                           out)
    with pytest.raises(ValueError, match="prepared"):  # tall: the iterate is the transpose
        newton_schulz_call(ortho, 1, 1024, 256, torch.empty(1, 1024, 256, dtype=torch.half),
                           None, torch.empty(1, 1024, 256, dtype=torch.bfloat16))


def _planned_launches(runs: list[tuple[int, int, int, int]]) -> int:
    """dionw_newton_schulz_group_launches for (kind, blocks, rows, cols) runs (wide)."""
    n = len(runs)

    def arr(ctype, values):
        return (ctype * max(n, 1))(*values)

    kinds, blocks = [r[0] for r in runs], [r[1] for r in runs]
    rows, cols = [r[2] for r in runs], [r[3] for r in runs]
    i64 = ctypes.c_int64
    return _lib.library().dionw_newton_schulz_group_launches(
        n, arr(ctypes.c_int32, kinds), arr(i64, blocks), arr(i64, rows), arr(i64, cols),
        arr(i64, rows), arr(i64, cols))


def test_queue_lanes() -> None:
    """How a flush spreads its calls over two streams: calls that share launches
    (one structure) stay on one lane, the structure with the most work on the
    first; calls that go out one by one are balanced by work; each lane keeps
    queue order."""
    from dionw_amd._matrix_step import _lanes
    from dionw_amd.newton_schulz import NewtonSchulzCall

    def call(kind, blocks, r, c, r_real=None, c_real=None):
        return NewtonSchulzCall(kind, blocks, r, c, 0, 0, r_real or r, c_real or c, 0, 0, c, r * c,
                                0, 0)

    wide = [call(0, 12, 768, 3072), call(0, 12, 768, 2304), call(0, 12, 768, 3072)]
    square = call(0, 12, 768, 768)
    # GPT-2 small: three wide Gram runs and the square run's standard iteration.
    assert _lanes([wide[0], square, wide[1], wide[2]], grouped=True) == [[0, 2, 3], [1]]
    assert _lanes(wide, grouped=True) == [[0, 1, 2]]      # one structure: one lane
    assert _lanes([square], grouped=True) == [[0]]
    # One by one: the biggest call alone, the other two together.
    big, small = call(0, 64, 1024, 4096), call(0, 32, 1024, 4096)
    assert _lanes([small, big, small], grouped=False) == [[1], [0, 2]]
    # A structure whose rows are not a multiple of 32 differs from one whose are.
    ragged = call(0, 12, 776, 3072, r_real=770)
    assert len(_lanes([wide[0], ragged], grouped=True)) == 2


def test_grouping_plan() -> None:
    """Which products the grouped call merges, from shapes alone (no GPU needed).

    A Gram run alone shares one launch between the independent Q Z and G Z
    products of its fourth iteration where that pays (17 of 18; not with an
    r = 352 side, which is not a multiple of 64). Llama-3-8B's four runs share
    their 14 symmetric and 2 syrk products (the Q X products already fill whole
    rounds alone); the MoE runs' products stay apart (their r = 352 side, and
    grouping the others would replace better-fitting 128 x 128 tiles); GPT-2's
    three Gram runs share every product and its square block keeps its own 15.
    """
    llama = [(0, 64, 1024, 4096), (0, 64, 256, 4096), (0, 64, 3584, 4096), (0, 32, 1024, 14336)]
    assert [_planned_launches([r]) for r in llama] == [17] * 4
    assert _planned_launches([(0, 28, 576, 1152)]) == 17
    assert _planned_launches([(0, 64, 352, 2048)]) == 18
    assert _planned_launches(llama) == 24
    assert _planned_launches([(0, 128, 352, 2048), (0, 64, 512, 1408)]) == 36
    gpt2 = [(0, 12, 768, 2304), (0, 12, 768, 768), (0, 12, 768, 3072), (0, 12, 768, 3072)]
    assert _planned_launches(gpt2) == 18 + 15
    assert _planned_launches([(1, 4, 256, 1024), (2, 4, 256, 1024)]) == 15  # both bf16 quintics
    assert _planned_launches([(7, 1, 64, 128)]) == -1
    assert _planned_launches([]) == 0


def test_missing_library_fails_loudly(monkeypatch, tmp_path) -> None:
    monkeypatch.setattr(_lib, "_PATH", tmp_path / "absent.so")
    monkeypatch.setattr(_lib, "_LIB", None)
    with pytest.raises(_lib.LibraryMissingError):
        _lib.library()


class _Tokens(nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.cls_token = nn.Parameter(torch.zeros(1, 1, 64))
        self.pos_embed = nn.Parameter(torch.zeros(1, 16, 64))


class _Net(nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.embed = nn.Embedding(100, 64)
        self.tokens = _Tokens()
        self.dw = nn.Conv2d(64, 64, 3, groups=64)
        self.conv = nn.Conv2d(64, 32, 3)
        self.fc = nn.Linear(64, 128)
        self.narrow = nn.Linear(64, 4)
        self.norm = nn.LayerNorm(64)


def test_default_route_table() -> None:
    groups, report = param_groups(_Net(), fraction=0.5, selection_min_dim=64)
    reasons = {p.name: (p.kind, p.reason) for p in report.parameters}
    assert reasons["embed.weight"] == (RouteKind.ADAMW, RouteReason.EMBEDDING)
    assert reasons["tokens.cls_token"] == (RouteKind.ADAMW, RouteReason.LEARNED_TOKENS)
    assert reasons["tokens.pos_embed"] == (RouteKind.ADAMW, RouteReason.EMBEDDING_NAME)
    assert reasons["dw.weight"] == (RouteKind.ADAMW, RouteReason.GROUPED_CONVOLUTION)
    assert reasons["conv.weight"] == (RouteKind.MATRIX, RouteReason.MATRIX)
    assert reasons["fc.weight"] == (RouteKind.MATRIX, RouteReason.MATRIX)
    assert reasons["fc.bias"] == (RouteKind.ADAMW, RouteReason.VECTOR)
    assert reasons["narrow.weight"] == (RouteKind.ADAMW, RouteReason.NARROW)
    assert reasons["norm.weight"] == (RouteKind.ADAMW, RouteReason.VECTOR)
    kinds = [g["dion_route"] for g in groups]
    assert kinds == sorted(kinds)  # adamw groups first
    fractions = {p.name: p.fraction for p in report.parameters}
    assert fractions["fc.weight"] == 0.5 and fractions["conv.weight"] == 1.0  # 32 < 64
    decay = {id(p): g.get("weight_decay") for g in groups for p in g["params"]}
    net_embed_decayed = [g for g in groups if any(p.shape == (100, 64) for p in g["params"])][0]
    assert "weight_decay" not in net_embed_decayed  # embeddings are decayed by default
    assert None in decay.values() and 0.0 in decay.values()
    lines = report.lines()
    assert lines[0] == "dionw parameter routing:"
    assert any("adamw (embedding): embed.weight (100, 64)" in line for line in lines)


def test_declared_routes_and_conflicts() -> None:
    net = _Net()
    groups, report = param_groups(net, routes={net.fc.weight: Route(RouteKind.MATRIX, num_heads=2)})
    entry = {p.name: p for p in report.parameters}["fc.weight"]
    assert entry.reason is RouteReason.DECLARED and entry.num_heads == 2
    with pytest.raises(ValueError, match="does not divide"):
        param_groups(net, routes={net.fc.weight: Route(RouteKind.MATRIX, num_heads=3)})
    with pytest.raises(ValueError, match="MATRIX route"):
        param_groups(net, routes={net.fc.bias: Route(RouteKind.MATRIX)})
    with pytest.raises(ValueError):
        Route(RouteKind.ADAMW, num_heads=2)
    with pytest.raises(ValueError):
        param_groups(net, fraction=0.0)


def test_ema_config_validation_and_kats() -> None:
    with pytest.raises(ValueError):
        EMAConfig(decay=1.0)
    with pytest.raises(ValueError):
        EMAConfig(decay_final=0.99)
    with pytest.raises(ValueError):
        EMAConfig(power_gamma=1.0, decay_final=0.99, decay_ramp_steps=10)
    ramp = EMAConfig(decay=0.9, decay_final=0.99, decay_ramp_steps=10)
    assert ramp.decay_at_step(0) == pytest.approx(0.9)
    assert ramp.decay_at_step(5) == pytest.approx(0.945)
    assert ramp.decay_at_step(20) == pytest.approx(0.99)
    power = EMAConfig(decay=0.999, power_gamma=6.94)
    assert power.decay_at_step(0) == 0.0
    assert power.decay_at_step(1) == 0.0
    assert power.decay_at_step(100) == pytest.approx(0.99 ** 7.94)
    assert power.decay_at_step(10**7) == pytest.approx(0.999)


def test_dion_rejects_cpu_and_unrouted_params() -> None:
    p = nn.Parameter(torch.zeros(8, 8))
    with pytest.raises(ValueError, match="CUDA"):
        dionw_amd.Dion([{"params": [p], "dion_route": "matrix"}], lr=1e-3)
    with pytest.raises(ValueError, match="lr and weight_decay"):
        dionw_amd.Dion([{"params": [p], "dion_route": "matrix"}], lr=-1.0)


def test_structural_key_refusal() -> None:
    saved = [{"dion_route": "matrix", "fraction": 0.25, "num_heads": None,
              "newton_schulz": "gram"}]
    current = [{"dion_route": "matrix", "fraction": 0.5, "num_heads": None,
                "newton_schulz": "gram", "row_normalization": "normuon",
                "momentum_form": "heavy_ball"}]
    with pytest.raises(ValueError, match="'fraction'"):
        refuse_structural_change(saved, current)
    current[0]["fraction"] = 0.25
    completed = refuse_structural_change(saved, current)
    # a checkpoint from before the update options is NorMuon with heavy-ball momentum
    assert completed[0]["row_normalization"] == "normuon"
    assert completed[0]["momentum_form"] == "heavy_ball"
    current[0]["momentum_form"] = "nesterov"
    with pytest.raises(ValueError, match="'momentum_form'"):
        refuse_structural_change(saved, current)
    with pytest.raises(ValueError, match="param groups"):
        refuse_structural_change(saved, current * 2)
    with pytest.raises(ValueError, match="'newton_schulz'"):
        refuse_structural_change([{"dion_route": "matrix", "fraction": 0.25, "num_heads": None}],
                                 current)


def test_integration_example_binds_the_header_signature() -> None:
    """The ctypes binding shown to maintainers declares as many arguments as the
    header's declaration of the same entry point."""
    import re
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    doc = (root / "INTEGRATION.md").read_text()
    header = (root / "include" / "dionw_hip.h").read_text()
    name, argtypes = re.search(r"lib\.(dionw_\w+)\.argtypes = \[(.*?)\]", doc, re.S).groups()
    declared = re.search(rf"\b{name}\((.*?)\);", header, re.S).group(1)
    depth, entries = 0, 1
    for ch in argtypes.strip().rstrip(","):
        depth += (ch == "(") - (ch == ")")
        entries += ch == "," and depth == 0
    assert entries == declared.count(",") + 1
