"""Pins of the CPU oracle (no GPU): each check is independent of the oracle's
own formula — float64 brute force, closed forms, torch's CPU ops, the exact
SVD polar factor, the reference's known-answer tables — and is chosen so that
a plausible mistake (a dropped term, a swapped coefficient, a wrong index)
fails it.
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import dion_ref
from tests import spectra
from tests.conftest import rel_fro

COEFFICIENTS = json.loads(
    (Path(__file__).resolve().parent / "golden" / "coefficients.json").read_text())


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


def test_coefficient_tables_equal_the_reference_literals() -> None:
    """Every row of the Gram, Polar Express and Keller tables against the
    literals of the reference's source (tests/golden/coefficients.json, parsed
    from _gram.py:24-37, _polar_express.py:28-36, _keller.py:20-22)."""
    fx = COEFFICIENTS
    s = fx["gram_safety"]
    folded = tuple((a / s, b / s**3, c / s**5) for a, b, c in fx["gram_unmodified"])
    assert len(folded) == 5
    assert dion_ref.GRAM_COEFFICIENTS == folded
    assert dion_ref.GRAM_RESTART_ITERATION == fx["gram_restart_iteration"]
    assert [list(r) for r in dion_ref.POLAR_EXPRESS_COEFFICIENTS] == fx["polar_express"]
    assert dion_ref.POLAR_EXPRESS_NORM_SAFETY == fx["polar_express_norm_safety"]
    assert [list(r) for r in dion_ref.KELLER_COEFFICIENTS] == fx["keller"]
    assert dion_ref.KELLER_NORM_SAFETY == fx["keller_norm_safety"]


@pytest.mark.parametrize("n", [256, 1024])
def test_standard_iteration_vs_float64_polynomial(n: int) -> None:
    """The standard iteration on square blocks (_gram.py:41-47) against the same
    five polynomials in float64. The bar is the rounding it performs: the bf16
    output alone is ~2.3e-3 relative (unit roundoff 2^-8 / sqrt 3), plus 15
    float16 roundings of the iterate's lines (2^-11 / sqrt 3 each) compounding
    through the iteration; a dropped term or a wrong coefficient is off by far
    more (>5e-2)."""
    x = torch.randn(1, n, n, generator=torch.Generator().manual_seed(10 + n))
    target = dion_ref.polynomial_float64(x, dion_ref.GRAM_COEFFICIENTS, 1.0)
    err = rel_fro(dion_ref.gram_polar_express(x, 1e-7).float(), target)
    bar = 2 ** -8 / math.sqrt(3) + 15 * 2 ** -11 / math.sqrt(3)
    assert err < bar, (err, bar)


@pytest.mark.parametrize("shape", [(2, 96, 256), (2, 256, 96), (1, 128, 128)])
def test_cublas_quintic_vs_float64_polynomial(shape) -> None:
    """quintic_cublas (_polar_express.py:43-71) for both tables against the
    float64 polynomial, and a tall block (iterated from the right) against the
    transposed wide block: the same products, so equal to the rounding.

    Rounding A A to bf16 before scaling it by c (15.9 in Polar Express's first
    step) costs accuracy: measured 0.020-0.035 from the float64 polynomial
    (Keller 0.015-0.017) where quintic_triton is at 0.010-0.016, so the bars are
    0.05 and 0.03; a dropped or swapped term is off by more than 0.3."""
    x = torch.randn(*shape, generator=torch.Generator().manual_seed(12))
    for table, safety, fn, bar in ((dion_ref.POLAR_EXPRESS_COEFFICIENTS,
                                    dion_ref.POLAR_EXPRESS_NORM_SAFETY, dion_ref.polar_express,
                                    0.05),
                                   (dion_ref.KELLER_COEFFICIENTS, dion_ref.KELLER_NORM_SAFETY,
                                    dion_ref.keller, 0.03)):
        wide = x if shape[-2] <= shape[-1] else x.mT
        target = dion_ref.polynomial_float64(wide, table, safety)
        if shape[-2] > shape[-1]:
            target = target.mT
        out = fn(x, 1e-7)
        assert out.dtype == torch.bfloat16 and out.shape == x.shape
        err = rel_fro(out.float(), target)
        assert err < bar, (fn.__name__, shape, err)
        if shape[-2] != shape[-1]:
            flipped = fn(x.mT.contiguous(), 1e-7).mT
            assert rel_fro(flipped.float(), out.float()) < 1e-2, (fn.__name__, shape)


@pytest.mark.parametrize("shape", [(1, 256, 1024), (2, 64, 256)])
def test_gram_vs_float64_polynomial(shape) -> None:
    """Gram rounding error vs the same polynomials in float64 (bench/precision.py:
    103-117); the reference reports 0.003 for Gaussian 256 x 1024 (README)."""
    x = torch.randn(*shape, generator=torch.Generator().manual_seed(0))
    target = dion_ref.polynomial_float64(x, dion_ref.GRAM_COEFFICIENTS, 1.0)
    err = rel_fro(dion_ref.gram_polar_express(x, 1e-7).float(), target)
    assert err < 0.006, err


@pytest.mark.parametrize("spectrum", spectra.SPECTRA[1:])
def test_spectrum_matrices_have_their_singular_values(spectrum) -> None:
    """The test matrices carry the singular values they are named for."""
    x = spectra.spectrum_matrix(spectrum)
    assert x.shape == (1, *spectra.SHAPE) and x.dtype == torch.float32
    got = torch.linalg.svdvals(x[0].double())
    want = spectra.singular_values(spectrum, spectra.SHAPE[0])
    assert torch.allclose(got, want, rtol=1e-3, atol=1e-6)


@pytest.mark.parametrize("spectrum", spectra.ILL_CONDITIONED)
def test_gram_restart_bounds_rounding_on_ill_conditioned_spectra(spectrum) -> None:
    """test_newton_schulz.py:79-92 and :137-148 on the oracle: with singular
    values spread over decades, Gram in float16 stays within 0.08 of its
    float64 polynomials because of the restart (without it the iterated Gram
    matrix compounds its rounding past 0.1), rounds less than Polar Express in
    bfloat16, and a bfloat16 input costs it more than 1.8x."""
    x = spectra.spectrum_matrix(spectrum)
    gram_target = dion_ref.polynomial_float64(x, dion_ref.GRAM_COEFFICIENTS, 1.0)
    pe_target = dion_ref.polynomial_float64(
        x, dion_ref.POLAR_EXPRESS_COEFFICIENTS, dion_ref.POLAR_EXPRESS_NORM_SAFETY)
    gram = rel_fro(dion_ref.gram_polar_express(x, 1e-7).float(), gram_target)
    no_restart = rel_fro(dion_ref.gram_polar_express(x, 1e-7, restart=None).float(), gram_target)
    bf16_input = rel_fro(dion_ref.gram_polar_express(x.bfloat16(), 1e-7).float(), gram_target)
    polar_express = rel_fro(dion_ref.polar_express(x, 1e-7).float(), pe_target)
    assert gram < 0.08, gram
    assert no_restart > 0.1, no_restart
    assert gram < polar_express, (gram, polar_express)
    assert bf16_input > 1.8 * gram, (bf16_input, gram)


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


def test_polar_express_triton_vs_float64_polynomial() -> None:
    x = torch.randn(1, 128, 512, generator=torch.Generator().manual_seed(4))
    target = dion_ref.polynomial_float64(
        x, dion_ref.POLAR_EXPRESS_COEFFICIENTS, dion_ref.POLAR_EXPRESS_NORM_SAFETY
    )
    assert rel_fro(dion_ref.polar_express_triton(x, 1e-7).float(), target) < 0.03


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


def _float64_muon_step(w, g, buf, v, lr, mu, beta2, wd, *, nesterov, normuon):
    """Every-row steps written as Keller Jordan's Muon writes them
    (tests/test_muon.py:104-115 of the reference): a momentum buffer
    ``buf = mu buf + g``, the input ``g + mu buf`` (Nesterov) or ``buf``, the
    exact polar factor, NorMuon or not, decoupled decay. Dion's state holds
    ``M = mu buf``, so the two agree when ``buf`` starts at ``M / mu``."""
    w, g, buf, v = (t.double().clone() for t in (w, g, buf, v))
    blocks, rows, cols = w.shape
    scale = lr * 0.2 * math.sqrt(max(rows, cols))
    for b in range(blocks):
        buf[b] = mu * buf[b] + g[b]
        u = g[b] + mu * buf[b] if nesterov else buf[b]
        o = dion_ref.exact_polar(u)
        if normuon:
            v[b] = v[b] + (1 - beta2) * ((o**2).mean(-1, keepdim=True) - v[b])
            n = o / (v[b].sqrt() + 1e-8)
            upd = n * (o.norm() / n.norm()) * -scale
        else:
            upd = o * -scale
        w[b] *= 1 - lr * wd
        w[b] += upd
    return w, buf, v


@pytest.mark.parametrize(("nesterov", "normuon"), [(False, True), (True, False), (False, False),
                                                   (True, True)])
def test_every_row_step_vs_float64_muon(nesterov: bool, normuon: bool) -> None:
    """step_blocks with k = rows (heavy ball or Nesterov, NorMuon or none)
    against the float64 Muon restatement, over three steps."""
    g = torch.Generator().manual_seed(13)
    w = torch.randn(2, 24, 40, generator=g) * 0.02
    m = torch.zeros_like(w)
    v = torch.zeros(2, 24, 1)
    buf = torch.zeros_like(w)
    w64, v64 = w.clone(), v.clone()
    exact = lambda x, eps: dion_ref.exact_polar(x).float()  # noqa: E731
    for _ in range(3):
        grads = torch.randn(2, 24, 40, generator=g)
        w64, buf, v64 = _float64_muon_step(w64, grads, buf, v64, 1e-3, 0.95, 0.95, 0.1,
                                           nesterov=nesterov, normuon=normuon)
        dion_ref.step_blocks(w, grads, m, v, k=24, lr=1e-3, mu=0.95, beta2=0.95, weight_decay=0.1,
                             normuon=normuon, nesterov=nesterov, orthogonalize=exact)
        assert rel_fro(m, 0.95 * buf) < 1e-6
        assert rel_fro(w, w64) < 1e-6
        if normuon:
            assert rel_fro(v, v64) < 1e-5


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
