"""Pins of the CPU oracle (no GPU): each check is independent of the oracle's
own formula — float64 brute force, closed forms, torch's CPU ops, the exact
SVD polar factor, the reference's known-answer tables — and is chosen so that
a plausible mistake (a dropped term, a swapped coefficient, a wrong index)
fails it.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import dion_ref
from tests.conftest import rel_fro


@pytest.mark.parametrize(("rows", "cols"), [(37, 3000), (8, 4096), (5, 1001), (3, 6), (2, 64)])
def test_row_l1_scores_vs_float64_brute_force(rows: int, cols: int) -> None:
    m = np.random.default_rng(0).standard_normal((rows, cols)).astype(np.float32)
    got = dion_ref.row_l1_scores(m)
    brute = np.abs(m.astype(np.float64)).sum(-1)
    np.testing.assert_allclose(got, brute, rtol=2e-6)
    # A dropped chunk or lane would show far above rounding.
    m2 = m.copy()
    m2[:, -1] += 1.0
    assert np.all(dion_ref.row_l1_scores(m2) != got)


def test_row_l1_scores_order_is_the_documented_tree() -> None:
    """Tiny case spelled out: 8 columns -> lanes 0 and 1 hold one float4 each."""
    m = np.arange(1, 9, dtype=np.float32)[None] * np.float32(0.1)
    a = np.abs(m[0])
    lane0 = (a[0] + a[1]) + (a[2] + a[3])
    lane1 = (a[4] + a[5]) + (a[6] + a[7])
    assert dion_ref.row_l1_scores(m)[0] == np.float32(lane0 + lane1)


def test_topk_rows_sets_and_ties() -> None:
    rng = np.random.default_rng(1)
    scores = rng.random(1000).astype(np.float32)
    k = 250
    expected = np.sort(np.argpartition(-scores.astype(np.float64), k - 1)[:k])
    assert np.array_equal(dion_ref.topk_rows(scores, k), expected)
    tied = np.zeros(10, np.float32)
    tied[[2, 7]] = 1.0
    assert np.array_equal(dion_ref.topk_rows(tied, 4), [0, 1, 2, 7])


def test_gram_coefficients_fold_the_safety_factor() -> None:
    a, b, c = dion_ref.GRAM_COEFFICIENTS[0]
    assert math.isclose(a * 1.05, 8.28721201814563)
    assert math.isclose(b * 1.05**3, -23.595886519098837)
    assert math.isclose(c * 1.05**5, 17.300387312530933)


@pytest.mark.parametrize("shape", [(1, 256, 1024), (2, 64, 256)])
def test_gram_vs_float64_polynomial(shape) -> None:
    """Gram rounding error vs the same polynomials in float64 (bench/precision.py:
    103-117); the reference reports 0.003 for Gaussian 256 x 1024 (README)."""
    x = torch.randn(*shape, generator=torch.Generator().manual_seed(0))
    target = dion_ref.polynomial_float64(x, dion_ref.GRAM_COEFFICIENTS, 1.0)
    err = rel_fro(dion_ref.gram_polar_express(x, 1e-7).float(), target)
    assert err < 0.006, err


@pytest.mark.parametrize("shape", [(3, 64, 256), (3, 256, 64), (3, 128, 128), (96, 160)])
def test_every_orthogonalization_near_exact_polar(shape) -> None:
    """test_newton_schulz.py:46-64 and :125-134: within 0.2 of the exact polar factor."""
    x = torch.randn(*shape, generator=torch.Generator().manual_seed(2))
    exact = dion_ref.exact_polar(x)
    for name, fn in dion_ref.ORTHOGONALIZE.items():
        out = fn(x, 1e-7)
        assert out.dtype == torch.bfloat16 and out.shape == x.shape
        bar = 0.3 if "keller" in name else 0.2
        assert rel_fro(out.float(), exact) < bar, name


def test_keller_singular_values_in_band() -> None:
    """test_muon.py:242-249: Keller's quintic leaves singular values in [0.6, 1.25]."""
    x = torch.randn(2, 64, 96, generator=torch.Generator().manual_seed(3))
    s = torch.linalg.svdvals(dion_ref.keller(x, 1e-7).double())
    assert float(s.min()) > 0.6 and float(s.max()) < 1.25


def test_polar_express_vs_float64_polynomial() -> None:
    x = torch.randn(1, 128, 512, generator=torch.Generator().manual_seed(4))
    target = dion_ref.polynomial_float64(
        x, dion_ref.POLAR_EXPRESS_COEFFICIENTS, dion_ref.POLAR_EXPRESS_NORM_SAFETY
    )
    assert rel_fro(dion_ref.polar_express(x, 1e-7).float(), target) < 0.03


def test_normalize_rows_closed_form() -> None:
    g = torch.Generator().manual_seed(5)
    o = torch.randn(2, 8, 16, generator=g).bfloat16()
    v = torch.rand(2, 8, 1, generator=g)
    step = torch.tensor(-0.01)
    out, new_v = dion_ref.normalize_rows(o, v, 0.95, step)
    u = o.double()
    v_ref = v.double() + 0.05 * ((u**2).mean(-1, keepdim=True) - v.double())
    n = u / (v_ref.sqrt() + 1e-8)
    ref = n * (u.norm(dim=(-2, -1), keepdim=True) / n.norm(dim=(-2, -1), keepdim=True)) * -0.01
    assert rel_fro(new_v, v_ref) < 1e-6
    assert rel_fro(out, ref) < 1e-6


def _float64_step(w, g, m, v, k, lr, mu, beta2, wd):
    """A second, loop-per-block float64 restatement of one selected-rows step
    with the exact polar factor (independent of dion_ref.step_blocks)."""
    w, g, m, v = (t.double().clone() for t in (w, g, m, v))
    blocks, rows, cols = w.shape
    scale = lr * 0.2 * math.sqrt(max(rows, cols)) * math.sqrt(min(rows, cols) / min(k, cols))
    for b in range(blocks):
        m[b] += g[b]
        order = sorted(range(rows), key=lambda r: (-float(m[b, r].abs().sum()), r))[:k]
        idx = torch.tensor(sorted(order))
        sel = m[b, idx].clone()
        m[b, idx] *= mu
        o = dion_ref.exact_polar(sel)
        v_sel = v[b, idx] + (1 - beta2) * ((o**2).mean(-1, keepdim=True) - v[b, idx])
        v[b, idx] = v_sel
        n = o / (v_sel.sqrt() + 1e-8)
        upd = n * (o.norm() / n.norm()) * -scale
        w[b] *= 1 - lr * wd
        w[b, idx] += upd
    return w, m, v


def test_step_blocks_vs_float64_restatement() -> None:
    g = torch.Generator().manual_seed(6)
    w = torch.randn(2, 24, 40, generator=g) * 0.02
    m = torch.zeros_like(w)
    v = torch.zeros(2, 24, 1)
    exact = lambda x, eps: dion_ref.exact_polar(x).float()  # noqa: E731
    for _ in range(3):
        grads = torch.randn(2, 24, 40, generator=g)
        w64, m64, v64 = _float64_step(w, grads, m, v, 6, 1e-3, 0.95, 0.95, 0.1)
        dion_ref.step_blocks(w, grads, m, v, k=6, lr=1e-3, mu=0.95, beta2=0.95, weight_decay=0.1,
                             orthogonalize=exact)
        assert rel_fro(m, m64) < 1e-6
        assert rel_fro(v, v64) < 1e-5
        assert rel_fro(w, w64) < 1e-6


def test_adamw_oracle_vs_torch_cpu() -> None:
    """ATen's fused AdamW on the CPU takes the same formula (float32 tolerance)."""
    rng = np.random.default_rng(7)
    p = rng.standard_normal(1000).astype(np.float32)
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    tp, tm, tv = (torch.from_numpy(a.copy()) for a in (p, m, v))
    steps = torch.zeros(())
    for step in range(1, 4):
        grad = (rng.standard_normal(1000) * 1e-3).astype(np.float32)
        dion_ref.adamw(p, grad, m, v, step, lr=3e-4, beta1=0.9, beta2=0.95, weight_decay=0.05,
                       eps=1e-8)
        steps += 1
        torch._fused_adamw_([tp], [torch.from_numpy(grad)], [tm], [tv], [], [steps], amsgrad=False,
                            lr=3e-4, beta1=0.9, beta2=0.95, weight_decay=0.05, eps=1e-8,
                            maximize=False, grad_scale=None, found_inf=None)
        np.testing.assert_allclose(p, tp.numpy(), rtol=1e-6, atol=1e-9)
        np.testing.assert_allclose(v, tv.numpy(), rtol=1e-6, atol=1e-18)


@pytest.mark.parametrize("decay", [0.9999, 0.3])
def test_ema_lerp_vs_torch_cpu(decay) -> None:
    rng = np.random.default_rng(8)
    s = rng.standard_normal(500).astype(np.float32)
    p = rng.standard_normal(500).astype(np.float32)
    ref = torch.from_numpy(s.copy()).lerp_(torch.from_numpy(p), 1.0 - decay).numpy()
    np.testing.assert_allclose(dion_ref.ema_lerp(s, p, decay), ref, rtol=2e-7, atol=1e-7)
    assert np.array_equal(dion_ref.ema_lerp(p, p, decay), p)
