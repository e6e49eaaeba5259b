"""``dionw_normuon_stats_noalloc`` against ``dionw_normuon_stats`` through the C ABI (GPU).

The no-allocation variant keeps its per-row partial sums in a device array of
the library instead of a caller workspace; its outputs (variance, row
denominators, block scales) must equal the workspace variant's bit for bit,
on two calls in a row (the second smaller, so stale contents of the shared
array would show), in selected-row and every-row mode. Oversized calls are
rejected before anything is launched.
"""

from __future__ import annotations

import pytest
import torch

from dionw_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _stats(noalloc: bool, o, idx, variance, blocks, k, rows, cols, beta2=0.95, step=-0.01):
    rowd = torch.empty(blocks, k, device=DEV)
    scale = torch.empty(blocks, device=DEV)
    stream = _lib.stream_handle(torch.device(DEV))
    idx_ptr = None if idx is None else idx.data_ptr()
    if noalloc:
        _lib.call("dionw_normuon_stats_noalloc", o.data_ptr(), blocks, k, rows, cols, idx_ptr,
                  variance.data_ptr(), beta2, step, rowd.data_ptr(), scale.data_ptr(), stream)
    else:
        partials = torch.empty(2 * blocks * k, device=DEV)
        _lib.call("dionw_normuon_stats", o.data_ptr(), blocks, k, rows, cols, idx_ptr,
                  variance.data_ptr(), beta2, step, rowd.data_ptr(), partials.data_ptr(),
                  scale.data_ptr(), stream)
    return rowd, scale


def _case(g: torch.Generator, blocks: int, rows: int, k: int, cols: int):
    o = torch.randn(blocks, k, cols, generator=g, device=DEV).bfloat16()
    variance = torch.rand(blocks, rows, generator=g, device=DEV) * 1e-3
    idx = None
    if k < rows:
        idx = torch.stack([torch.randperm(rows, generator=g, device=DEV)[:k].sort().values
                           for _ in range(blocks)]).to(torch.int32)
    return o, idx, variance


@pytest.mark.parametrize(("first", "second"), [
    ((64, 14336, 3584, 4096), (3, 100, 30, 70)),     # selected rows, then a smaller call
    ((8, 512, 512, 1024), (2, 64, 64, 96)),          # every row, then a smaller call
])
def test_noalloc_stats_equal_workspace_stats(first, second) -> None:
    g = torch.Generator(device=DEV).manual_seed(17)
    for blocks, rows, k, cols in (first, second):
        print(f"[no_alloc] blocks={blocks} rows={rows} k={k} cols={cols}", flush=True)
        o, idx, variance = _case(g, blocks, rows, k, cols)
        v_ws, v_na = variance.clone(), variance.clone()
        rowd_ws, scale_ws = _stats(False, o, idx, v_ws, blocks, k, rows, cols)
        rowd_na, scale_na = _stats(True, o, idx, v_na, blocks, k, rows, cols)
        torch.cuda.synchronize()
        assert torch.equal(v_na, v_ws), f"variance {blocks}x{rows}x{k}x{cols}"
        assert torch.equal(rowd_na, rowd_ws), f"row denominators {blocks}x{rows}x{k}x{cols}"
        assert torch.equal(scale_na, scale_ws), f"block scales {blocks}x{rows}x{k}x{cols}"


def test_noalloc_stats_reject_oversized_calls() -> None:
    o = torch.empty(8, device=DEV, dtype=torch.bfloat16)
    rowd = torch.empty(1, device=DEV)
    with pytest.raises(ValueError, match="device scratch"):
        _lib.call("dionw_normuon_stats_noalloc", o.data_ptr(), 2, 2**19, 2**19, 8, None,
                  rowd.data_ptr(), 0.95, -0.01, rowd.data_ptr(), rowd.data_ptr(),
                  _lib.stream_handle(torch.device(DEV)))
