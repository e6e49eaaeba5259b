"""Rounding of the HIP Newton-Schulz kinds on well- and ill-conditioned inputs.

Mirrors tests/test_newton_schulz.py:46-148 of the reference: each kind's
rounding error is its relative Frobenius distance to the same polynomials
evaluated in float64 on the float32 input (bench/precision.py:103-117). The HIP
Gram iteration must round no worse than the oracle's restatement of the
reference's (the same float16 steps, restart at iteration 2), stay within 0.08
on singular values spread over decades, beat bfloat16 Polar Express there, and
lose precision when fed a bfloat16 input.
"""

from __future__ import annotations

import pytest
import torch

from dionw_amd.newton_schulz import NewtonSchulz, newton_schulz_fn
from oracle import dion_ref
from tests import spectra
from tests.conftest import rel_fro

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
EPS = 1e-7


def _hip(kind: NewtonSchulz, x: torch.Tensor) -> torch.Tensor:
    out = newton_schulz_fn(kind)(x.to(DEV), EPS)
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16 and out.shape == x.shape
    return out.cpu().float()


def _gram_target(x: torch.Tensor) -> torch.Tensor:
    return dion_ref.polynomial_float64(x, dion_ref.GRAM_COEFFICIENTS, 1.0)


def _polar_express_target(x: torch.Tensor) -> torch.Tensor:
    return dion_ref.polynomial_float64(
        x, dion_ref.POLAR_EXPRESS_COEFFICIENTS, dion_ref.POLAR_EXPRESS_NORM_SAFETY)


@pytest.mark.parametrize("spectrum", spectra.SPECTRA)
def test_gram_rounds_like_the_reference_iteration(spectrum: str) -> None:
    """test_newton_schulz.py:67-76: the HIP Gram iteration's rounding error is
    within 1.3x (+3e-3) of the reference iteration's, here its oracle
    restatement, on every spectrum."""
    x = spectra.spectrum_matrix(spectrum)
    target = _gram_target(x)
    ours = rel_fro(_hip(NewtonSchulz.GRAM, x), target)
    reference = rel_fro(dion_ref.gram_polar_express(x, EPS).float(), target)
    assert ours < 1.3 * reference + 3e-3, (spectrum, ours, reference)


@pytest.mark.parametrize("spectrum", spectra.ILL_CONDITIONED)
def test_gram_restart_bounds_the_rounding_error(spectrum: str) -> None:
    """test_newton_schulz.py:79-92: on ill-conditioned inputs the HIP Gram
    iteration (float16, restart at 2) stays within 0.08 of its polynomials and
    rounds less than the HIP Polar Express iterations in bfloat16."""
    x = spectra.spectrum_matrix(spectrum)
    gram = rel_fro(_hip(NewtonSchulz.GRAM, x), _gram_target(x))
    assert gram < 0.08, (spectrum, gram)
    for kind in (NewtonSchulz.POLAR_EXPRESS, NewtonSchulz.POLAR_EXPRESS_TRITON):
        quintic = rel_fro(_hip(kind, x), _polar_express_target(x))
        assert gram < quintic, (spectrum, kind.value, gram, quintic)


@pytest.mark.parametrize("spectrum", spectra.ILL_CONDITIONED)
def test_float32_input_keeps_gram_precise_on_ill_conditioned_inputs(spectrum: str) -> None:
    """test_newton_schulz.py:137-148: a bfloat16 input (as microsoft/dion passes
    it) costs the Gram iteration at least 1.8x its rounding error where the
    singular values spread over decades; the HIP path reads float32 directly."""
    x = spectra.spectrum_matrix(spectrum)
    target = _gram_target(x)
    float32_input = rel_fro(_hip(NewtonSchulz.GRAM, x), target)
    bfloat16_input = rel_fro(_hip(NewtonSchulz.GRAM, x.bfloat16()), target)
    assert bfloat16_input > 1.8 * float32_input, (spectrum, bfloat16_input, float32_input)


WIDE_TALL_SQUARE = [(3, 64, 256), (3, 256, 64), (3, 128, 128)]


@pytest.mark.parametrize("shape", WIDE_TALL_SQUARE)
def test_gram_lands_as_close_to_the_polar_factor_as_polar_express(shape) -> None:
    """test_newton_schulz.py:46-64: Gram lands as close to the exact polar
    factor as Polar Express, in wide (Gram), tall (transposed) and square
    (standard iteration) orientation."""
    x = torch.randn(*shape, generator=torch.Generator().manual_seed(0))
    exact = dion_ref.exact_polar(x)
    gram = _hip(NewtonSchulz.GRAM, x)
    polar_express = _hip(NewtonSchulz.POLAR_EXPRESS, x)
    gram_error = rel_fro(gram, exact)
    polar_express_error = rel_fro(polar_express, exact)
    assert gram_error < 0.2, gram_error
    assert gram_error < polar_express_error + 0.02, (gram_error, polar_express_error)
    assert rel_fro(gram, polar_express) < 0.15
