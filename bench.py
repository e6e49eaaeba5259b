"""Benchmark of the Dion optimizer step on one MI355X.

Default workload: one full ``Dion.step()`` over
Llama-3-8B-shaped float32 parameters — 32 layers of q/o 4096x4096, k/v
1024x4096, gate/up 14336x4096, down 4096x14336 on Dion with fraction 0.25,
embedding and lm_head 128256x4096 plus the RMSNorm weights on AdamW — with
synthetic weights ~0.02 N(0,1) and gradients ~1e-3 N(0,1) resident in HBM.

Prints one JSON line: the step time (``value``, ms), the Gram Newton-Schulz
TFLOP/s and momentum-pass GB/s measured live with HIP events on the stream
the kernels run on, the roofline of the dominant kernel family (the
Newton-Schulz MFMA products) and the CPU oracle's time on a bounded sample.

Usage: python bench.py [--steps K] [--warmup W] [--config NAME] [--no-cpu-baseline]
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time
from collections import defaultdict
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_MFMA_TFLOPS = 2500.0   # MI355X dense fp16/bf16
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E

LLAMA = {
    "layers": 32,
    "matrices": [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
                 ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)],
    "vocab": 128256,
    "hidden": 4096,
}
GPT2 = {
    "layers": 12,
    "matrices": [("qkv", 2304, 768), ("proj", 768, 768), ("fc", 3072, 768), ("fc2", 768, 3072)],
    "vocab": 50257,
    "hidden": 768,
}


def ns_flops(kind: int, r: int, c: int) -> float:
    """Algorithmic FLOPs of one Newton-Schulz block r x c (r <= c): the Gram
    iteration 6 r^2 c + 23 r^3, the standard / quintic 15 r^2 c + 5 r^3."""
    if kind == 0 and c > r:
        return 6.0 * r * r * c + 23.0 * r**3
    return 15.0 * r * r * c + 5.0 * r**3


class Timeline:
    """HIP-event timing of the library's entry points (instrumented steps only)."""

    def __init__(self) -> None:
        import torch

        self.torch = torch
        self.events: list[tuple[str, dict, object, object]] = []

    def wrap(self, lib_module) -> None:
        original = lib_module.call
        torch = self.torch

        def timed(name, *args):
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            original(name, *args)
            end.record()
            self.events.append((name, {"args": args}, start, end))

        lib_module.call = timed
        self._restore = (lib_module, original)

    def unwrap(self) -> None:
        module, original = self._restore
        module.call = original

    def summary(self) -> dict[str, dict[str, float]]:
        """Per entry point: calls, algorithmic flops or bytes, and "ms", the time
        during which at least one of its calls ran. The optimizer may run calls
        on two streams at once, so their durations are not summed: each call's
        interval is placed on one clock (the first event's) and the union is
        measured."""
        self.torch.cuda.synchronize()
        out: dict[str, dict[str, float]] = defaultdict(lambda: {"ms": 0.0, "calls": 0, "flops": 0.0,
                                                                 "bytes": 0.0})
        spans: dict[str, list[tuple[float, float]]] = defaultdict(list)
        origin = self.events[0][2] if self.events else None
        for name, meta, start, end in self.events:
            key = "dionw_newton_schulz" if name == "dionw_newton_schulz_group" else name
            spans[key].append((origin.elapsed_time(start), origin.elapsed_time(end)))
            entry = out[name]
            entry["calls"] += 1
            a = meta["args"]
            if name == "dionw_newton_schulz":
                kind, batch, r, c, r_real, c_real = a[0], a[1], a[2], a[3], a[6], a[7]
                entry["flops"] += batch * ns_flops(kind, r_real, c_real)
                # The library's own count of the product launches of the call.
                one = lambda t, v: (t * 1)(v)
                entry["launches"] = entry.get("launches", 0) + self._restore[0].library(
                ).dionw_newton_schulz_group_launches(
                    1, one(ctypes.c_int32, kind), one(ctypes.c_int64, batch), one(ctypes.c_int64, r),
                    one(ctypes.c_int64, c), one(ctypes.c_int64, r_real), one(ctypes.c_int64, c_real))
            elif name == "dionw_newton_schulz_group":
                # Reported with the single calls: the same products, grouped.
                del out[name]
                entry = out["dionw_newton_schulz"]
                entry["calls"] += 1
                n = a[0]
                for i in range(n):
                    entry["flops"] += a[2][i] * ns_flops(a[1][i], a[7][i], a[8][i])
                # The library's own count of the products it launched for the call.
                launches = self._restore[0].library().dionw_newton_schulz_group_launches(
                    n, a[1], a[2], a[3], a[4], a[7], a[8])
                entry["launches"] = entry.get("launches", 0) + launches
            elif name == "dionw_accumulate_scores":
                count, rows, cols = a[1], a[2], a[3]
                entry["bytes"] += 12.0 * count * rows * cols
            elif name == "dionw_prepare_ns_input":
                # per element: M read (if any) and written (write_m), G read in
                # every-row mode (no idx), the 16-bit (or float32) input in each
                # orientation written
                momentum, idx, blocks, cols, k = a[2], a[3], a[5], a[7], a[8]
                write_m, elem, rowmajor, transposed = a[13], a[14], a[15], a[16]
                out_bytes = 4.0 if elem == 2 else 2.0
                per = ((4.0 if momentum else 0.0) + (4.0 if momentum and write_m else 0.0)
                       + (4.0 if idx is None else 0.0)
                       + out_bytes * ((1 if rowmajor else 0) + (1 if transposed else 0)))
                entry["bytes"] += per * blocks * k * cols
            elif name == "dionw_apply_update":
                count, bpt, rows, cols, k, decay_on = a[1], a[2], a[3], a[4], a[5], a[13]
                n = count * bpt * rows * cols
                s = count * bpt * k * cols
                entry["bytes"] += (8.0 * n if decay_on else 8.0 * s) + 2.0 * s
            elif name == "dionw_apply_update_ema":
                # every row: W read, S read and written; W written where it changes
                count, bpt, rows, cols, k, decay_on = a[2], a[3], a[4], a[5], a[6], a[14]
                n = count * bpt * rows * cols
                s = count * bpt * k * cols
                entry["bytes"] += 12.0 * n + (4.0 * n if decay_on else 4.0 * s) + 2.0 * s
            elif name == "dionw_adamw":
                entry["bytes"] += 28.0 * sum(a[5][i] for i in range(a[6]))
            elif name == "dionw_adamw_ema":
                entry["bytes"] += 36.0 * sum(a[6][i] for i in range(a[7]))
            elif name == "dionw_ema_update":
                entry["bytes"] += (8.0 if a[5] else 12.0) * sum(a[2][i] for i in range(a[3]))
        for key, intervals in spans.items():
            out[key]["ms"] = covered_ms(intervals)
        return dict(out)


def covered_ms(intervals: list[tuple[float, float]]) -> float:
    """Length of the union of (begin, end) intervals: the time during which at
    least one of them was running."""
    covered, reach = 0.0, float("-inf")
    for begin, finish in sorted(intervals):
        if finish > reach:
            covered += finish - max(begin, reach)
            reach = finish
    return covered


def build_llama(torch, dev, spec, fraction):
    g = torch.Generator(device=dev).manual_seed(0)
    hidden = spec["hidden"]

    def param(*shape):
        p = torch.nn.Parameter(torch.empty(*shape, device=dev).normal_(0.0, 0.02, generator=g))
        p.grad = torch.empty_like(p).normal_(0.0, 1e-3, generator=g)
        return p

    matrices, norms = [], []
    for _ in range(spec["layers"]):
        for _, rows, cols in spec["matrices"]:
            matrices.append(param(rows, cols))
        norms.extend([param(hidden), param(hidden)])
    norms.append(param(hidden))
    embed = [param(spec["vocab"], hidden), param(spec["vocab"], hidden)]
    groups = [
        {"params": embed, "dion_route": "adamw"},
        {"params": norms, "dion_route": "adamw", "weight_decay": 0.0},
        {"params": matrices, "dion_route": "matrix", "fraction": fraction},
    ]
    n_params = sum(p.numel() for grp in groups for p in grp["params"])
    return groups, n_params


def build_gpt2(torch, dev):
    """GPT-2 small (124 M parameters). Every linear is Dion with fraction 0.25 and
    selection_min_dim 1024, so with their 768-wide sides all update every row;
    LayerNorm weights/biases, linear biases, wte 50257x768 and wpe 1024x768 take AdamW."""
    g = torch.Generator(device=dev).manual_seed(0)

    def param(*shape):
        p = torch.nn.Parameter(torch.empty(*shape, device=dev).normal_(0.0, 0.02, generator=g))
        p.grad = torch.empty_like(p).normal_(0.0, 1e-3, generator=g)
        return p

    matrices, vectors = [], []
    for _ in range(GPT2["layers"]):
        for _, rows, cols in GPT2["matrices"]:
            matrices.append(param(rows, cols))
            vectors.append(param(rows))                      # linear bias
        vectors.extend(param(768) for _ in range(4))         # two LayerNorms
    vectors.extend([param(768), param(768)])                 # final LayerNorm
    embed = [param(50257, 768), param(1024, 768)]
    groups = [
        {"params": embed + vectors, "dion_route": "adamw", "weight_decay": 0.0},
        {"params": matrices, "dion_route": "matrix", "fraction": 1.0},
    ]
    return groups, sum(p.numel() for grp in groups for p in grp["params"])


def build_moe(torch, dev):
    """MoE expert stack: 64 experts with fp32 gate/up 1408x2048 and down 2048x1408
    (separate 2-D parameters), gradients 1e-3 * Student-t(df=3)."""
    g = torch.Generator(device=dev).manual_seed(0)

    def student_t(*shape):
        z = torch.empty(*shape, device=dev).normal_(generator=g)
        chi2 = sum(torch.empty(*shape, device=dev).normal_(generator=g) ** 2 for _ in range(3))
        return z / torch.sqrt(chi2 / 3.0) * 1e-3

    def param(*shape):
        p = torch.nn.Parameter(torch.empty(*shape, device=dev).normal_(0.0, 0.02, generator=g))
        p.grad = student_t(*shape)
        return p

    experts = []
    for _ in range(64):
        experts += [param(1408, 2048), param(1408, 2048), param(2048, 1408)]
    return experts, sum(p.numel() for p in experts)


def gram_ns_bench(torch, steps: int, warmup: int) -> dict:
    """Standalone Gram Newton-Schulz on 16 bf16 blocks 1024x4096,
    entries N(0,1) pre-normalized by their Frobenius norm, 5 iterations."""
    from dionw_amd.newton_schulz import NewtonSchulz, newton_schulz_fn

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.empty(16, 1024, 4096, device=dev).normal_(generator=g)
    x = (x / torch.linalg.vector_norm(x, dim=(-2, -1), keepdim=True)).bfloat16()
    fn = newton_schulz_fn(NewtonSchulz.GRAM)
    for _ in range(warmup):
        fn(x, 1e-8)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(steps):
        fn(x, 1e-8)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    flops = 16 * ns_flops(0, 1024, 4096)
    tflops = flops / (ms * 1e-3) / 1e12
    return {
        "metric": "Gram Newton-Schulz ms, 16 x 1024x4096 bf16 (config 2)",
        "value": round(ms, 4), "unit": "ms", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "f16 MFMA (bf16 input)", "data": "synthetic",
        "config": {"workload": "gram-ns: 16 blocks 1024x4096, 5 iterations, restart at 2"},
        "gram_ns_tflops": round(tflops, 1),
        "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": PEAK_MFMA_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / PEAK_MFMA_TFLOPS, 4),
                     "traffic": None},
    }


# The reference's README performance table (bench/optimizer_step.py:40-196):
# a pre-norm transformer of width 2048, depth 24, 16 heads and a 32000-token
# vocabulary (1.34 G parameters), random gradients 1e-3 N(0,1), lr 1e-4,
# betas (0.9, 0.95), no weight decay; only ``step()`` is timed, as the median
# of 20 single-step timings after 5 warm-up steps.
TRANSFORMER = {"width": 2048, "depth": 24, "heads": 16, "vocab": 32000}
TABLE_WARMUP, TABLE_TIMED = 5, 20
# Published step times of the default rule at f=0.25 (README.md:491-507).
TRANSFORMER_PUBLISHED_MS = {"RTX 4090": 92.5, "RTX 5090": 61.0, "GH200": 27.2}
# The wide blocks of the reference's Newton-Schulz table (bench/newton_schulz.py:19-24).
WIDE_SHAPES = ((28, 576, 1152), (28, 576, 4608), (28, 1152, 4608), (16, 1024, 8192))


def median_step_ms(torch, call, warmup: int = TABLE_WARMUP, timed: int = TABLE_TIMED) -> float:
    """Median GPU time of ``call`` over ``timed`` calls timed one by one with
    events on the current stream, after ``warmup`` untimed calls."""
    import statistics

    for _ in range(warmup):
        call()
    torch.cuda.synchronize()
    samples = []
    for _ in range(timed):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        call()
        end.record()
        end.synchronize()
        samples.append(start.elapsed_time(end))
    return statistics.median(samples)


def build_transformer(torch, dev):
    """The README table's transformer on ``dev`` with a gradient on every
    parameter; each block declares its fused QKV projection as 3 * heads
    separate matrices."""
    import dionw_amd

    nn = torch.nn
    spec = TRANSFORMER

    class Block(nn.Module):
        def __init__(self, width: int, heads: int) -> None:
            super().__init__()
            self.heads = heads
            self.norm1, self.norm2 = nn.LayerNorm(width), nn.LayerNorm(width)
            self.qkv = nn.Linear(width, 3 * width)
            self.proj = nn.Linear(width, width)
            self.fc1 = nn.Linear(width, 4 * width)
            self.fc2 = nn.Linear(4 * width, width)

        def dion_routes(self):
            return ((self.qkv.weight,
                     dionw_amd.Route(dionw_amd.RouteKind.MATRIX, num_heads=3 * self.heads)),)

    class Transformer(nn.Module):
        def __init__(self) -> None:
            super().__init__()
            self.embed = nn.Embedding(spec["vocab"], spec["width"])
            self.blocks = nn.ModuleList(Block(spec["width"], spec["heads"])
                                        for _ in range(spec["depth"]))
            self.norm = nn.LayerNorm(spec["width"])
            self.head = nn.Linear(spec["width"], spec["vocab"], bias=False)

    torch.manual_seed(0)
    with torch.device(dev):
        model = Transformer()
    for param in model.parameters():
        param.grad = torch.randn_like(param) * 1e-3
    return model


def transformer_table(torch) -> dict:
    """Step time of each optimizer of the README table on one MI355X, and the
    host dispatch time of the default step."""
    import gc

    import dionw_amd

    dev = torch.device("cuda:0")

    def dion(model, fraction, selection_min_dim, kind):
        groups, _ = dionw_amd.param_groups(model, fraction=fraction,
                                           selection_min_dim=selection_min_dim, min_matrix_dim=8)
        return dionw_amd.Dion(groups, lr=1e-4, betas=(0.9, 0.95), weight_decay=0.0,
                              matrix_update=dionw_amd.MatrixUpdate(
                                  newton_schulz=kind,
                                  row_normalization=dionw_amd.RowNormalization.NORMUON,
                                  momentum_form=dionw_amd.MomentumForm.HEAVY_BALL))

    ns = dionw_amd.NewtonSchulz
    variants = {
        "dionw, f=0.25, default rule": lambda m: dion(m, 0.25, 1024, ns.GRAM),
        "dionw, f=0.25, every block, Gram": lambda m: dion(m, 0.25, 1, ns.GRAM),
        "dionw, f=0.25, every block, Polar Express Triton":
            lambda m: dion(m, 0.25, 1, ns.POLAR_EXPRESS_TRITON),
        "dionw, f=0.5, default rule": lambda m: dion(m, 0.5, 1024, ns.GRAM),
        "fused AdamW (torch), all parameters":
            lambda m: torch.optim.AdamW(m.parameters(), lr=1e-4, betas=(0.9, 0.95), fused=True),
    }
    table, host, n_params = {}, None, 0
    for name, make in variants.items():
        print(f"[bench] transformer-1.34b: {name}", file=sys.stderr, flush=True)
        model = build_transformer(torch, dev)
        n_params = sum(p.numel() for p in model.parameters())
        opt = make(model)
        table[name] = round(median_step_ms(torch, opt.step), 3)
        if host is None:
            host = host_dispatch_ms(torch, opt, samples=TABLE_TIMED)
        del opt, model
        gc.collect()
        torch.cuda.empty_cache()
    value = table["dionw, f=0.25, default rule"]
    return {
        "metric": "Dion step ms, 1.34B transformer, f=0.25 default rule (README table)",
        "value": value, "unit": "ms", "n_gpus": 1, "steps": TABLE_TIMED, "warmup": TABLE_WARMUP,
        "ms_per_step": value, "higher_is_better": False, "scaling": "weak",
        # Against the GH200 figure of README.md:507 (lower is better).
        "vs_baseline": round(value / TRANSFORMER_PUBLISHED_MS["GH200"], 4),
        "dtype": "f32 state, f16 MFMA Newton-Schulz", "data": "synthetic",
        "config": {"workload": "transformer-1.34b: width 2048, depth 24, 16 heads, vocab 32000, "
                               "QKV split per head, default routing; median of 20 steps",
                   "params": n_params},
        "variants_ms": table,
        "host_dispatch_ms": round(host, 3),
        "published_ms": TRANSFORMER_PUBLISHED_MS,
    }


def wide_ns_table(torch) -> dict:
    """Gram Newton-Schulz against both Polar Express variants on the reference's
    wide blocks: median ms of one batched call on a float32 N(0,1) batch."""
    from dionw_amd.newton_schulz import NewtonSchulz, newton_schulz_fn

    dev = torch.device("cuda:0")
    kinds = (NewtonSchulz.GRAM, NewtonSchulz.POLAR_EXPRESS_TRITON, NewtonSchulz.POLAR_EXPRESS)
    rows = []
    for shape in WIDE_SHAPES:
        torch.manual_seed(0)
        x = torch.randn(*shape, device=dev)
        ms = {kind.value: median_step_ms(torch, lambda k=kind: newton_schulz_fn(k)(x, 1e-7))
              for kind in kinds}
        blocks, r, c = shape
        gram = ms[NewtonSchulz.GRAM.value]
        rows.append({
            "shape": "x".join(map(str, shape)),
            "ms": {k: round(v, 4) for k, v in ms.items()},
            "gram_tflops": round(blocks * ns_flops(0, r, c) / (gram * 1e-3) / 1e12, 1),
            "speedup_vs_triton": round(ms[NewtonSchulz.POLAR_EXPRESS_TRITON.value] / gram, 3),
            "speedup_vs_cublas": round(ms[NewtonSchulz.POLAR_EXPRESS.value] / gram, 3),
        })
        print(f"[bench] ns-wide {rows[-1]}", file=sys.stderr, flush=True)
    worst = min(row["speedup_vs_triton"] for row in rows)
    return {
        "metric": "Gram NS speedup over Polar Express (Triton products), wide blocks, minimum",
        "value": worst, "unit": "x", "n_gpus": 1, "steps": TABLE_TIMED, "warmup": TABLE_WARMUP,
        "ms_per_step": None, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16 MFMA (Gram), bf16 MFMA (Polar Express)", "data": "synthetic",
        "config": {"workload": "ns-wide: " + ", ".join(r["shape"] for r in rows)},
        "rows": rows,
        # README.md:536-539: RTX 4090 / RTX 5090 / GH200.
        "published_speedup_vs_triton": ["1.2-1.9", "1.3-2.7", "1.05-1.8"],
        "published_speedup_vs_cublas": ["1.5-2.5", "1.9-3.5", "1.1-2.2"],
    }


def cpu_share() -> dict:
    """The host CPUs this process may use: the affinity set, capped by a cgroup
    CPU quota (a GPU box grants each job a share of a larger host), with the
    host's own count and CPU model for the record."""
    cpus = os.cpu_count() or 1
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else cpus
    quota = None
    try:
        fields = Path("/sys/fs/cgroup/cpu.max").read_text().split()
        if fields and fields[0] != "max":
            quota = max(1, int(int(fields[0]) // int(fields[1])))
    except (OSError, ValueError, IndexError):
        pass
    if quota is not None:
        usable = min(usable, quota)
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"threads": usable, "host_cpus": cpus, "cgroup_quota_cpus": quota, "cpu_model": model}


def cpu_baseline(spec, fraction: float, share: dict) -> dict:
    """The CPU oracle on one decoder layer's Dion blocks plus 1/layers of the
    AdamW elements, scaled by the layer count (labelled extrapolated): one
    warm-up step, then the median of three timed steps, on every usable core."""
    import statistics

    import numpy as np
    import torch

    from oracle import dion_ref

    threads = share["threads"]
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)
    blocks = []
    for _, rows, cols in spec["matrices"]:
        w = torch.randn(1, rows, cols, generator=g) * 0.02
        blocks.append((w, torch.randn(1, rows, cols, generator=g) * 1e-3, torch.zeros_like(w),
                       torch.zeros(1, rows, 1), rows))
    adamw_numel = (2 * spec["vocab"] * spec["hidden"]) // spec["layers"] + 2 * spec["hidden"]
    rng = np.random.default_rng(0)
    ap = (rng.standard_normal(adamw_numel) * 0.02).astype(np.float32)
    ag = (rng.standard_normal(adamw_numel) * 1e-3).astype(np.float32)
    am, av = np.zeros_like(ap), np.zeros_like(ap)

    def one_layer(step: int) -> None:
        for w, grad, m, v, rows in blocks:
            k = min(rows, math.ceil(fraction * rows))
            dion_ref.step_blocks(w, grad, m, v, k=k, lr=3e-4, mu=0.95, beta2=0.95,
                                 weight_decay=0.05, kind="gram")
        dion_ref.adamw(ap, ag, am, av, float(step), lr=3e-4, beta1=0.9, beta2=0.95,
                       weight_decay=0.05, eps=1e-8)

    t0 = time.perf_counter()
    one_layer(1)  # warm-up
    samples = []
    for step in range(2, 5):
        t1 = time.perf_counter()
        one_layer(step)
        samples.append(time.perf_counter() - t1)
    per_layer = statistics.median(samples)
    return {
        "value": per_layer * spec["layers"] * 1e3,
        "unit": "ms/step (extrapolated)",
        "cores": threads,
        "host_cpus": share["host_cpus"],
        "cgroup_quota_cpus": share["cgroup_quota_cpus"],
        "cpu_model": share["cpu_model"],
        "kind": "port",
        "sample": f"oracle (torch CPU restatement, {threads} threads): one decoder layer's Dion "
                  f"blocks + 1/{spec['layers']} of the AdamW elements; 1 warm-up step, median "
                  f"of 3 steps, x{spec['layers']} layers",
        "sample_seconds": round(time.perf_counter() - t0, 2),
    }


# Busy-wait queued ahead of each dispatch sample: ~0.1 s at MI355X clocks, far
# longer than a step's host work, so the host never waits on the GPU.
GPU_BUSY_CYCLES = 200_000_000


def host_dispatch_ms(torch, opt, samples: int = 7, call=None) -> float:
    """Median host time of one ``opt.step()`` (or ``call``) while the GPU is
    held busy (reference bench/host_dispatch.py:28-56): the Python and launch
    overhead alone, independent of how many steps are timed."""
    import statistics

    call = opt.step if call is None else call
    times = []
    for _ in range(samples):
        torch.cuda.synchronize()
        torch.cuda._sleep(GPU_BUSY_CYCLES)
        start = time.perf_counter()
        call()
        times.append((time.perf_counter() - start) * 1e3)
    torch.cuda.synchronize()
    return statistics.median(times)


def step_graph_report(torch, opt, steps: int) -> dict:
    """A ``StepGraph`` of the optimizer against its eager steps, same process:
    GPU ms per step of each (HIP events, three alternating rounds of ``steps``)
    and the host ms of one call with the GPU held busy."""
    from dionw_amd import StepGraph

    graph = StepGraph(opt)
    graph.replay()

    def timed(call) -> float:
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
        for _ in range(steps):
            call()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / steps

    rounds = [(timed(opt.step), timed(graph.replay)) for _ in range(3)]
    return {
        "eager_ms": [round(e, 3) for e, _ in rounds],
        "replay_ms": [round(r, 3) for _, r in rounds],
        "eager_host_ms": round(host_dispatch_ms(torch, opt), 3),
        "replay_host_ms": round(host_dispatch_ms(torch, opt, call=graph.replay), 3),
    }


TRAFFIC_FILE = ROOT / "profiles" / "traffic.json"


# The Newton-Schulz runs of one Llama-3-8B step: (blocks, selected rows, cols).
LLAMA_NS_RUNS = [(64, 1024, 4096), (64, 256, 4096), (64, 3584, 4096), (32, 1024, 14336)]


def ns_algorithmic_bytes(blocks: int, r: int, c: int) -> float:
    """HBM bytes the 18 products of one Gram iteration must move for a run of
    ``blocks`` r x c blocks (16-bit data; per product each operand read once,
    each output written once): 2 syrks (X read, G written), 5 polynomials (G
    read, Z written; twice Q = Z + aI too), 3 Q and 6 Gram updates (two
    operands read, one written) and 2 Q X products (Q and X read, X written):
    6 r c + 43 r^2 elements per block. Where r is not a multiple of 32 the Q X
    products read X^T instead and the restart writes X^T too: 7 r c."""
    return 2.0 * blocks * ((6.0 if r % 32 == 0 else 7.0) * r * c + 43.0 * r * r)


def traffic_bytes():
    """Average HBM bytes per Newton-Schulz product launch of the Llama-3-8B
    step, from the committed FETCH_SIZE / WRITE_SIZE measurement (``--probe``
    under rocprofv3 --pmc), or None."""
    try:
        data = json.loads(TRAFFIC_FILE.read_text())
        return data["ns_step"]["hbm_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def state_bytes(opt) -> int:
    """Bytes of the optimizer's state tensors (each storage once: bucket views
    share their bucket's storage)."""
    seen: dict[int, int] = {}
    for state in opt.state.values():
        for value in state.values():
            if hasattr(value, "untyped_storage") and value.is_cuda:
                storage = value.untyped_storage()
                seen[storage.data_ptr()] = storage.nbytes()
    return sum(seen.values())


def memory_report(torch, opt, before_optimizer: int) -> dict:
    """The step's device memory above the parameters, gradients and optimizer
    state, from torch's allocator: ``scratch_held_gb`` is what the HIP passes
    keep between steps (named scratch buffers, regrown on demand), and
    ``peak_above_state_gb`` the peak of one more step above parameters,
    gradients and state (held scratch included) — the figure the reference
    quotes for its runs (src/dionw/_matrix_step.py:44-49)."""
    from dionw_amd import _workspace

    torch.cuda.synchronize()
    state = state_bytes(opt)
    held = _workspace.held_bytes()
    torch.cuda.reset_peak_memory_stats()
    opt.step()
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated()
    return {
        "state_gb": round(state / 1e9, 3),
        "scratch_held_gb": round(held / 1e9, 3),
        "peak_above_state_gb": round((peak - before_optimizer - state) / 1e9, 3),
        "device_peak_gb": round(peak / 1e9, 3),
    }


def probe() -> int:
    """The launches whose traffic is measured (run under ``rocprofv3 --pmc``): a
    copy of known size for calibrating the counters, the grouped Newton-Schulz
    call of one Llama-3-8B step (its 24 product launches) and one accumulate
    pass over a gate/up-sized run."""
    import torch

    from dionw_amd import _lib
    from dionw_amd.newton_schulz import (
        NewtonSchulz,
        newton_schulz_call,
        newton_schulz_fn,
        prepared_orientations,
        run_newton_schulz_group,
    )

    dev = torch.device("cuda:0")
    src = torch.empty(256 * 2**20, device=dev)  # 1 GiB of float32
    dst = torch.empty_like(src)
    dst.copy_(src)
    ortho = newton_schulz_fn(NewtonSchulz.GRAM)
    calls, buffers = [], []
    for i, (blocks, r, c) in enumerate(LLAMA_NS_RUNS):
        x = (torch.randn(blocks, r, c, device=dev) / math.sqrt(r * c)).half()
        # Like the optimizer step, only the inputs the iteration reads.
        xt = x.mT.contiguous() if prepared_orientations(r, c)[1] else None
        out = torch.empty(blocks, r, c, device=dev, dtype=torch.bfloat16)
        buffers += [x, xt, out]
        calls.append(newton_schulz_call(ortho, blocks, r, c, x, xt, out, f"probe_ns#{i}"))
    run_newton_schulz_group(calls, _lib.stream_handle(dev))
    del buffers
    grads = [torch.randn(14336, 4096, device=dev) * 1e-3 for _ in range(18)]
    mom = torch.zeros(18 * 14336, 4096, device=dev)
    scores = torch.empty(18 * 14336, device=dev)
    rowsq = torch.empty_like(scores)
    _lib.call("dionw_accumulate_scores", _lib.ptr_array(grads), 18, 14336, 4096, mom.data_ptr(),
              scores.data_ptr(), rowsq.data_ptr(), _lib.F16, _lib.stream_handle(dev))
    torch.cuda.synchronize()
    print("probe done: copy 1 GiB, grouped Newton-Schulz of the Llama-3-8B runs, "
          "accumulate 18x14336x4096")
    return 0


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--probe", action="store_true",
                        help="run the counter-calibration launches and exit")
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=5)
    parser.add_argument("--warmup", type=int, default=2)
    parser.add_argument("--config", default="llama3-8b",
                        choices=["llama3-8b", "gpt2-small", "gram-ns", "moe", "moe-muon",
                                 "transformer-1.34b", "ns-wide"])
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--instrumented-steps", type=int, default=2)
    parser.add_argument("--step-graph", action="store_true",
                        help="also time replays of the step recorded as a HIP graph (no EMA)")
    args = parser.parse_args()
    if args.probe:
        return probe()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (the optimizer step is single-device); "
              f"--gpus {args.gpus} is not supported", file=sys.stderr)
        return 2

    import torch

    import dionw_amd
    from dionw_amd import _lib

    if args.config == "gram-ns":
        print(json.dumps(gram_ns_bench(torch, args.steps, args.warmup)), flush=True)
        return 0
    if args.config == "transformer-1.34b":
        print(json.dumps(transformer_table(torch)), flush=True)
        return 0
    if args.config == "ns-wide":
        print(json.dumps(wide_ns_table(torch)), flush=True)
        return 0
    dev = torch.device("cuda:0")
    spec = LLAMA if args.config == "llama3-8b" else GPT2
    fraction = 0.25
    print(f"[bench] building {args.config} parameters", file=sys.stderr, flush=True)
    kwargs = {}
    if args.config == "llama3-8b":
        groups, n_params = build_llama(torch, dev, spec, fraction)
    elif args.config == "gpt2-small":
        groups, n_params = build_gpt2(torch, dev)
    else:
        experts, n_params = build_moe(torch, dev)
        if args.config == "moe":
            groups = [{"params": experts, "dion_route": "matrix", "fraction": fraction}]
            kwargs["ema"] = dionw_amd.EMAConfig(decay=0.9999, update_every_n_steps=1)
        else:
            groups = [{"params": experts, "dion_route": "matrix", "fraction": 1.0}]
            kwargs["matrix_update"] = dionw_amd.MUON_UPDATE
    torch.cuda.synchronize()
    before_optimizer = torch.cuda.memory_allocated()  # parameters and gradients
    opt = dionw_amd.Dion(groups, lr=3e-4, weight_decay=0.05, momentum=0.95, muon_beta2=0.95,
                         betas=(0.9, 0.95), eps=1e-8, **kwargs)
    torch.cuda.synchronize()
    print(f"[bench] {n_params / 1e9:.2f} G params; warmup {args.warmup}", file=sys.stderr,
          flush=True)
    for _ in range(args.warmup):
        opt.step()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    print(f"[bench] timing {args.steps} steps", file=sys.stderr, flush=True)
    start.record()
    for _ in range(args.steps):
        opt.step()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps
    host_dispatch = host_dispatch_ms(torch, opt)

    timeline = Timeline()
    timeline.wrap(_lib)
    for _ in range(args.instrumented_steps):
        opt.step()
    summary = timeline.summary()
    timeline.unwrap()
    div = max(args.instrumented_steps, 1)
    ns = summary.get("dionw_newton_schulz", {"ms": 0.0, "flops": 0.0, "calls": 0})
    ns_tflops = ns["flops"] / (ns["ms"] * 1e-3) / 1e12 if ns["ms"] else 0.0
    acc = summary.get("dionw_accumulate_scores", {"ms": 0.0, "bytes": 0.0})
    acc_gbs = acc["bytes"] / (acc["ms"] * 1e-3) / 1e9 if acc["ms"] else 0.0
    phases = {name: {"ms_per_step": round(v["ms"] / div, 3), "calls_per_step": v["calls"] // div,
                     **({"tflops": round(v["flops"] / (v["ms"] * 1e-3) / 1e12, 1)} if v["flops"] else {}),
                     **({"gbs": round(v["bytes"] / (v["ms"] * 1e-3) / 1e9, 1)} if v["bytes"] else {})}
              for name, v in sorted(summary.items(), key=lambda kv: -kv[1]["ms"])}
    print(f"[bench] phases {json.dumps(phases)}", file=sys.stderr, flush=True)
    memory = memory_report(torch, opt, before_optimizer)
    print(f"[bench] memory {json.dumps(memory)}", file=sys.stderr, flush=True)
    graph = None
    if args.step_graph:
        if opt.ema is not None:
            print("[bench] --step-graph: the EMA config cannot be recorded; skipped",
                  file=sys.stderr, flush=True)
        else:
            graph = step_graph_report(torch, opt, args.steps)
            print(f"[bench] step graph {json.dumps(graph)}", file=sys.stderr, flush=True)

    cpu = None
    if not args.no_cpu_baseline and args.config == "llama3-8b":
        print("[bench] CPU oracle baseline", file=sys.stderr, flush=True)
        cpu = cpu_baseline(spec, fraction, cpu_share())

    line = {
        "metric": {
            "llama3-8b": "Dion step ms at Llama-3-8B shapes",
            "gpt2-small": "Dion step ms at GPT-2-small shapes (config 3)",
            "moe": "Dion step ms, MoE 64 experts + GPU EMA (config 5a)",
            "moe-muon": "Muon step ms, MoE 64 experts (config 5b)",
        }[args.config],
        "value": round(ms, 3),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 state, f16/bf16 MFMA Newton-Schulz",
        "data": "synthetic",
        "config": {
            "workload": {
                "llama3-8b": f"llama3-8b: full Dion step (Dion f={fraction} on every linear, "
                             "AdamW on embeddings/lm_head/norms), fp32 params resident in HBM",
                "gpt2-small": "gpt2-small: Dion on every linear (all rows: min side 768 < 1024), "
                              "AdamW on LayerNorms, biases, wte, wpe",
                "moe": "moe: 64 experts gate/up 1408x2048 + down 2048x1408, Dion f=0.25, "
                       "GPU EMA 0.9999 every step, Student-t(3) gradients",
                "moe-muon": "moe-muon: the same experts with MUON_UPDATE (Keller bf16, Nesterov, "
                            "every row)",
            }[args.config],
            "params": n_params,
        },
        "gram_ns_tflops": round(ns_tflops, 1),
        "momentum_pass_gbs": round(acc_gbs, 1),
        # The momentum pass (M += G with the row scores; 12 B per element) against
        # the HBM roofline.
        "momentum_roofline": {"bound": "hbm", "achieved": round(acc_gbs, 1),
                              "peak": PEAK_HBM_GBS, "unit": "GB/s",
                              "frac": round(acc_gbs / PEAK_HBM_GBS, 4)} if acc_gbs else None,
        "host_dispatch_ms": round(host_dispatch, 3),
        "memory": memory,
        **({"step_graph": graph} if graph is not None else {}),
        "phases": phases,
        "roofline": {
            "bound": "mfma",
            "kernel": "gemm_nt_pipe_group_kernel / gemm_nt_pipe_kernel (Newton-Schulz products)",
            "achieved": round(ns_tflops, 1),
            "peak": PEAK_MFMA_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(ns_tflops / PEAK_MFMA_TFLOPS, 4),
            # Measured for the Llama-3-8B gate/up product only; other workloads'
            # dominant launches have other shapes.
            "traffic": traffic_bytes() if args.config == "llama3-8b" else None,
            "avg_launch_us": round(ns["ms"] * 1e3 / max(ns.get("launches", 0), 1), 1),
            "launches_per_step": ns.get("launches", 0) // div,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
