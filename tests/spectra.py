"""Test matrices with prescribed singular values (shared by the oracle and GPU
tests of Newton-Schulz rounding).

The spectra are those the reference measures rounding on (bench/precision.py:
31-101): a 256 x 1024 matrix ``U diag(s) V^T`` with orthonormal ``U`` and
``V`` from float64 QR of seeded Gaussian matrices, ``s`` decaying geometrically
over 2, 4 or 6 decades, or 8 values at 1 over a floor of 1e-3 or 1e-4; plus a
plain Gaussian matrix. Momentum matrices are often close to low rank, which is
where rounding errors in an iterated Gram matrix compound. The matrices are
built on the CPU with torch's CPU generator, so they are the same on every
host.
"""

from __future__ import annotations

import torch

SHAPE = (256, 1024)
LOW_RANK = 8
SPECTRA = ("gaussian", "geometric_2", "geometric_4", "geometric_6", "low_rank_3", "low_rank_4")
ILL_CONDITIONED = ("geometric_4", "geometric_6", "low_rank_3", "low_rank_4")


def singular_values(spectrum: str, count: int) -> torch.Tensor:
    """``count`` float64 singular values of ``spectrum``, largest first."""
    kind, _, decades = spectrum.rpartition("_")
    if kind == "geometric":
        return torch.logspace(0, -int(decades), count, dtype=torch.float64)
    if kind == "low_rank":
        values = torch.full((count,), 10.0 ** -int(decades), dtype=torch.float64)
        values[:LOW_RANK] = 1.0
        return values
    raise ValueError(f"{spectrum} has no prescribed singular values")


def spectrum_matrix(spectrum: str) -> torch.Tensor:
    """A seeded float32 ``[1, 256, 1024]`` CPU matrix with ``spectrum``."""
    rows, cols = SHAPE
    generator = torch.Generator().manual_seed(0)
    if spectrum == "gaussian":
        return torch.randn(1, rows, cols, generator=generator)
    left, _ = torch.linalg.qr(torch.randn(rows, rows, dtype=torch.float64, generator=generator))
    right, _ = torch.linalg.qr(torch.randn(cols, rows, dtype=torch.float64, generator=generator))
    return ((left * singular_values(spectrum, rows)) @ right.mT).float()[None]
