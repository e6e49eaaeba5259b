"""bench.py's contract pieces that need no GPU (CPU).

The FLOP convention of the Newton-Schulz TFLOP/s (F = 6 r^2 c + 23 r^3 for a
wide Gram block, 15 r^2 c + 5 r^3 for the others; not the MFMA work of the
upper-tile products), the products' algorithmic bytes behind
roofline.traffic, and the refusal of more than one GPU.
"""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import bench

ROOT = Path(__file__).resolve().parents[1]


def test_ns_flops_convention() -> None:
    # Gram iteration on a wide block: 2 syrks r^2 c, 5 symmetric polynomials r^3,
    # 3 Q updates 2 r^3, 3 Gram updates 4 r^3, 2 Q X products 2 r^2 c.
    r, c = 1024, 4096
    assert bench.ns_flops(0, r, c) == 2 * r * r * c + 5 * r**3 + 3 * 2 * r**3 + 3 * 4 * r**3 \
        + 2 * 2 * r * r * c
    # Square Gram blocks and the quintics: five rounds of syrk r^2 c, polynomial
    # r^3 and left product 2 r^2 c.
    assert bench.ns_flops(0, r, r) == 5 * (r * r * r + r**3 + 2 * r * r * r)
    assert bench.ns_flops(1, 1408, 2048) == 5 * (1408**2 * 2048 + 1408**3 + 2 * 1408**2 * 2048)
    # The gram-ns workload (the plugin call on 16 blocks 1024 x 4096): 0.8075 TFLOP.
    assert abs(16 * bench.ns_flops(0, 1024, 4096) / 1e12 - 0.8075) < 5e-4


def test_phase_time_is_the_union_of_call_intervals() -> None:
    """Calls on two streams overlap: a phase's time counts each instant once."""
    assert bench.covered_ms([]) == 0.0
    assert bench.covered_ms([(0.0, 2.0), (1.0, 3.0), (5.0, 6.0)]) == 4.0
    assert bench.covered_ms([(0.0, 10.0), (2.0, 3.0)]) == 10.0          # nested
    assert bench.covered_ms([(4.0, 5.0), (0.0, 1.0), (1.0, 2.0)]) == 3.0  # unsorted, touching
    assert bench.covered_ms([(1.0, 2.0), (1.0, 2.0)]) == 1.0            # identical


def test_ns_algorithmic_bytes() -> None:
    # Writes 18 r^2 + 2 r c, reads 25 r^2 + 4 r c per block (16-bit) when X is
    # read as it lies; a transposed copy adds one r c write.
    r, c = 1024, 4096
    assert bench.ns_algorithmic_bytes(1, r, c) == 2 * (6 * r * c + 43 * r * r)
    assert bench.ns_algorithmic_bytes(1, 1000, c) == 2 * (7 * 1000 * c + 43 * 1000**2)


def test_more_than_one_gpu_is_refused() -> None:
    out = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], cwd=ROOT,
                         capture_output=True, text=True, timeout=120)
    assert out.returncode != 0
    assert "one GPU" in out.stdout + out.stderr
