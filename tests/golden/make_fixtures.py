"""Write the golden fixtures of tests/test_golden.py from the CPU oracle.

The reference cannot run in this container (it needs CUDA and an installed
package), so the vectors come from the oracle's restatement of its PyTorch path
(oracle/dion_ref.py), on CPU-seeded inputs that the tests regenerate:

- ``small_step.npz``: three Dion steps of two 48x80 blocks, fraction 0.25,
  weight decay 0.1, Newton-Schulz replaced by the exact polar factor of the
  input (as tests/test_optimizer.py:90-132 does), so the GPU must match to
  float32 rounding; scores, indices, momentum, variance and weights per step.
- ``config1.npz``: one step of a 1024x1024 fp32 weight
  ~N(0, 0.02^2), gradient ~N(0, 1e-3^2), zero momentum, seed 0, fraction 1
  (NorMuon, the standard iteration of Gram Newton-Schulz on a square block),
  momentum 0.95, muon_beta2 0.95, lr 3e-4, weight decay 0.05: the variance, a
  64x64 corner of the updated weight, norms, and the whole update
  ``W_new - W (1 - lr wd)`` as float16 of update / max|update| (quantization
  ~3e-4 relative Frobenius, far below the 1e-2 bar it is held to).

Usage: python tests/golden/make_fixtures.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import dion_ref  # noqa: E402


def small_inputs():
    g = torch.Generator().manual_seed(1234)
    w = torch.randn(2, 48, 80, generator=g) * 0.02
    grads = torch.randn(3, 2, 48, 80, generator=g)
    return w, grads


def config1_inputs():
    g = torch.Generator().manual_seed(0)
    w = torch.randn(1024, 1024, generator=g) * 0.02
    grad = torch.randn(1024, 1024, generator=g) * 1e-3
    return w, grad


def exact_polar(x: torch.Tensor, epsilon: float) -> torch.Tensor:
    del epsilon
    return dion_ref.exact_polar(x).to(torch.bfloat16)


def small_expected():
    w, grads = small_inputs()
    m = torch.zeros_like(w)
    v = torch.zeros(2, 48, 1)
    out = {"w0": w.numpy().copy()}
    for step in range(3):
        res = dion_ref.step_blocks(w, grads[step], m, v, k=12, lr=1e-3, mu=0.95, beta2=0.95,
                                   weight_decay=0.1, orthogonalize=exact_polar)
        out[f"scores{step}"] = res.scores.astype(np.float32)
        out[f"index{step}"] = res.index.astype(np.int32)
        out[f"momentum{step}"] = m.numpy().copy()
        out[f"variance{step}"] = v.numpy().copy()
        out[f"weight{step}"] = w.numpy().copy()
    return out


def config1_expected():
    w, grad = config1_inputs()
    start = w.clone()
    m = torch.zeros(1, 1024, 1024)
    v = torch.zeros(1, 1024, 1)
    wb = w[None].clone()
    dion_ref.step_blocks(wb, grad[None], m, v, k=1024, lr=3e-4, mu=0.95, beta2=0.95,
                         weight_decay=0.05, kind="gram")
    update = wb[0] - start * (1.0 - 3e-4 * 0.05)
    scale = float(update.abs().max())
    return {
        "update_f16": (update / scale).numpy().astype(np.float16),
        "update_scale": np.float64(scale),
        "variance": v[0, :, 0].numpy().copy(),
        "weight_corner": wb[0, :64, :64].numpy().copy(),
        "update_norm": np.float64(update.double().norm()),
        "weight_norm": np.float64(wb[0].double().norm()),
        "momentum_abs_sum": np.float64(m.double().abs().sum()),
    }


def main() -> None:
    np.savez(HERE / "small_step.npz", **small_expected())
    np.savez_compressed(HERE / "config1.npz", **config1_expected())
    print("wrote", HERE / "small_step.npz", HERE / "config1.npz")


if __name__ == "__main__":
    main()
