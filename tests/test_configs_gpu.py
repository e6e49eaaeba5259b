"""The BASELINE configurations at their own shapes, HIP path against the oracle (GPU).

Each test runs the shapes, bucket sizes and hyperparameters ``bench.py`` times,
so that the kernels behind the reported numbers (tile sizes, grouped launches,
XCD run dealing) are the ones checked. Inputs are drawn on the GPU from seeded
generators and copied to the host, so the oracle sees the same bits. Where the
CPU oracle would take minutes (Llama-3-8B's 64-block buckets, MoE-Muon's 192
quintics) it runs on sampled blocks: blocks never interact, so a sample is
checked exactly as the whole would be.

Bars (the north star's, with the build's update-level bar): row selection and
momentum bit-exact; the update ``W_new - W d`` within ``1.6 e + 3e-3``
relative Frobenius of the oracle's, where ``e`` is the oracle's own
Newton-Schulz rounding error on the same input (its distance to the same
polynomials in float64); parameters within 2e-3; AdamW and the EMA bit-exact
against torch's own fused AdamW and ``_foreach_lerp_``. The configurations run
their full step counts (configs 3 and 5: 10 steps; config 4: 5 steps over all
32 layers): every block's momentum is checked at every step on the GPU (every
row is either ``M + G`` or ``fp32((M + G) mu)``, exactly ``k`` decayed rows per
block), and two sampled blocks per bucket against the oracle, from the GPU's
state before the step.
"""

from __future__ import annotations

import math

import pytest
import torch
from torch import nn

from dionw_amd import (
    FRACTION_KEY,
    MUON_UPDATE,
    ROUTE_KEY,
    Dion,
    EMAConfig,
    NewtonSchulz,
    _kernels,
    _lib,
    _workspace,
)
from dionw_amd.newton_schulz import (
    group_launches,
    newton_schulz_call,
    newton_schulz_fn,
    run_newton_schulz_call,
    run_newton_schulz_group,
)
from oracle import dion_ref
from tests.conftest import rel_fro

pytestmark = pytest.mark.gpu
DEV = "cuda"
LR, WD, MU, BETA2 = 3e-4, 0.05, 0.95, 0.95


def _say(msg: str) -> None:
    print(f"[configs] {msg}", flush=True)


def _normal(g: torch.Generator, *shape: int, std: float = 1.0) -> torch.Tensor:
    return torch.empty(*shape, device=DEV).normal_(0.0, std, generator=g)


def _student_t(g: torch.Generator, *shape: int) -> torch.Tensor:
    """1e-3 * Student-t with 3 degrees of freedom (z / sqrt(chi2_3 / 3))."""
    z = _normal(g, *shape)
    chi2 = sum(_normal(g, *shape) ** 2 for _ in range(3))
    return z / torch.sqrt(chi2 / 3.0) * 1e-3


def _check_run(name: str, params: list[nn.Parameter], opt: Dion, before: torch.Tensor,
               w_ref: torch.Tensor, mom_ref: torch.Tensor, var_ref: torch.Tensor,
               update_bar: float) -> None:
    """GPU state of ``params`` (stacked into [blocks, rows, cols]) against the
    oracle's after the same step from the same state ``before``."""
    shape = w_ref.shape
    got_m = torch.stack([opt.state[p]["momentum"].cpu() for p in params]).view(shape)
    assert torch.equal(got_m, mom_ref), f"{name}: momentum differs (row selection?)"
    got_w = torch.stack([p.detach().cpu() for p in params]).view(shape)
    decay = 1.0 - LR * WD
    err = rel_fro(got_w - before * decay, w_ref - before * decay)
    assert err < update_bar, f"{name}: update rel err {err}"
    assert rel_fro(got_w, w_ref) < 2e-3, f"{name}: parameters"
    got_v = torch.stack([opt.state[p]["variance"].cpu() for p in params]).view(var_ref.shape)
    assert rel_fro(got_v, var_ref) < 2e-2, f"{name}: NorMuon variance"


POLYNOMIALS = {"gram": (dion_ref.GRAM_COEFFICIENTS, 1.0),
               "keller_triton": (dion_ref.KELLER_COEFFICIENTS, dion_ref.KELLER_NORM_SAFETY)}


def _recording_oracle(kind: str, seen: dict):
    """The oracle's orthogonalization of ``kind``, recording its rounding error
    (distance to the same polynomials in float64) in ``seen["rounding"]``."""
    def ortho(x: torch.Tensor, epsilon: float) -> torch.Tensor:
        out = dion_ref.ORTHOGONALIZE[kind](x, epsilon)
        tall = x.shape[-2] > x.shape[-1]
        target = dion_ref.polynomial_float64(x.mT if tall else x, *POLYNOMIALS[kind])
        seen["rounding"] = max(seen.get("rounding", 0.0),
                               rel_fro(out.float(), target.mT if tall else target))
        return out
    return ortho


def _momentum_of(opt: Dion, p: nn.Parameter) -> torch.Tensor:
    """A parameter's momentum before its first step is zero."""
    m = opt.state[p].get("momentum")
    return torch.zeros_like(p) if m is None else m.detach().clone()


def _check_every_block(name: str, params: list[nn.Parameter], opt: Dion,
                       m_old: list[torch.Tensor], k: int) -> None:
    """Every block's momentum on the GPU: ``s = M + G`` (one exact float32
    add); a selected row is ``fp32(s mu)``, every other row ``s``, and each
    block decays exactly ``k`` rows (a row equal both ways, all zero, counts
    either way)."""
    mu = torch.tensor(MU, dtype=torch.float32, device=DEV)
    for i, (p, m0) in enumerate(zip(params, m_old)):
        m_new = opt.state[p]["momentum"]
        total = m0 + p.grad
        is_decayed = (m_new == total * mu).all(-1)
        is_kept = (m_new == total).all(-1)
        assert bool((is_decayed | is_kept).all()), f"{name} block {i}: a row is neither"
        only_decayed = int((is_decayed & ~is_kept).sum())
        either = int((is_decayed & is_kept).sum())
        assert only_decayed <= k <= only_decayed + either, (
            f"{name} block {i}: {only_decayed} decayed rows, expected {k}")


def _check_sampled(name: str, params: list[nn.Parameter], opt: Dion, sample: list[int],
                   before: dict, k: int, kind: str = "gram", normuon: bool = True,
                   nesterov: bool = False) -> None:
    """The sampled blocks' step against the oracle, from the GPU's state
    ``before`` the step (weights, momentum, variance, gradient of each)."""
    w = torch.stack([before[i][0] for i in sample])
    mom = torch.stack([before[i][1] for i in sample])
    var = torch.stack([before[i][2] for i in sample])
    grad = torch.stack([before[i][3] for i in sample])
    start = w.clone()
    seen: dict = {}
    dion_ref.step_blocks(w, grad, mom, var, k=k, lr=LR, mu=MU, beta2=BETA2, weight_decay=WD,
                         kind=kind, normuon=normuon, nesterov=nesterov,
                         orthogonalize=_recording_oracle(kind, seen))
    got_m = torch.stack([opt.state[params[i]]["momentum"].cpu() for i in sample])
    assert torch.equal(got_m, mom), f"{name}: momentum of blocks {sample} differs"
    got_w = torch.stack([params[i].detach().cpu() for i in sample])
    decay = 1.0 - LR * WD
    err = rel_fro(got_w - start * decay, w - start * decay)
    bar = 1.6 * seen["rounding"] + 3e-3
    assert err < bar, f"{name}: update rel err {err}, bar {bar} (blocks {sample})"
    assert rel_fro(got_w, w) < 2e-3, f"{name}: parameters of blocks {sample}"
    if normuon:
        got_v = torch.stack([opt.state[params[i]]["variance"].cpu() for i in sample])
        assert rel_fro(got_v, var) < 2e-2, f"{name}: NorMuon variance of blocks {sample}"


def _state_before(opt: Dion, params: list[nn.Parameter], sample: list[int]) -> dict:
    """(weights, momentum, variance, gradient) of the sampled blocks, on the host."""
    out = {}
    for i in sample:
        p = params[i]
        var = opt.state[p].get("variance")
        var = torch.zeros(p.shape[0], 1) if var is None else var.detach().cpu().clone()
        out[i] = (p.detach().cpu().clone(), _momentum_of(opt, p).cpu(), var.view(-1, 1),
                  p.grad.detach().cpu().clone())
    return out


def _sample(n: int, step: int) -> list[int]:
    """Two distinct blocks of ``n`` that move with the step."""
    a = (7 * step) % n
    b = (n - 1 - 3 * step) % n
    return [a, b] if a != b else [a, (a + 1) % n]


# ---- products at the tile counts that switch on XCD run dealing ---------------

@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_products_with_xcd_run_dealing(dtype: torch.dtype) -> None:
    """256x256 products with 64 or more tiles per batch entry deal their tiles to
    the XCDs in runs of 32: 16 x 2048^2 (64 tiles) against float32 matmul, and
    the symmetric 4 x 3584^2 product (105 upper tiles) against float32 and bit
    for bit against the full product of the same symmetric matrix."""
    _say(f"xcd-dealt products {dtype}")
    g = torch.Generator(device=DEV).manual_seed(21)
    a = (_normal(g, 16, 2048, 2048) / 45).to(dtype)
    b = (_normal(g, 16, 2048, 2048) / 45).to(dtype)
    d = _normal(g, 16, 2048, 2048).to(dtype)
    out = _kernels.gemm_nt(a, b, d=d, alpha=0.7, beta=-1.3)
    expected = 0.7 * (a.float() @ b.float().mT) - 1.3 * d.float()
    torch.cuda.synchronize()
    tol = 2e-3 if dtype == torch.float16 else 1e-2
    err = rel_fro(out.float(), expected)
    assert err < tol, f"16 x 2048^2 {dtype}: rel err {err}"
    x = (_normal(g, 4, 3584, 3584) / 85).to(dtype)
    s = (x + x.mT).contiguous()
    sym = _kernels.gemm_nt(s, s, d=s, alpha=0.5, beta=-1.5, symmetric=True)
    full = _kernels.gemm_nt(s, s, d=s, alpha=0.5, beta=-1.5, symmetric=False)
    ref = 0.5 * (s.float() @ s.float()) - 1.5 * s.float()
    torch.cuda.synchronize()
    assert torch.equal(sym, full), f"4 x 3584^2 {dtype}: symmetric and full products differ"
    err = rel_fro(sym.float(), ref)
    assert err < tol, f"4 x 3584^2 {dtype}: rel err {err}"


# ---- config 2: standalone Gram Newton-Schulz, 16 x 1024 x 4096 bf16 ------------

def test_config2_gram_newton_schulz_batch16_bf16() -> None:
    """The config-2 call (16 bf16 blocks of 1024 x 4096, each divided by its
    Frobenius norm) against the oracle on every block, and its rounding error
    against the float64 polynomial on two blocks."""
    _say("config 2: gram-ns 16 x 1024 x 4096 bf16")
    g = torch.Generator(device=DEV).manual_seed(0)
    x = _normal(g, 16, 1024, 4096)
    x = (x / torch.linalg.vector_norm(x, dim=(-2, -1), keepdim=True)).bfloat16()
    out = newton_schulz_fn(NewtonSchulz.GRAM)(x, 1e-8)
    torch.cuda.synchronize()
    x_cpu, out_cpu = x.cpu(), out.cpu().float()
    ref = dion_ref.gram_polar_express(x_cpu, 1e-8).float()
    err = rel_fro(out_cpu, ref)
    assert err < 1e-2, f"config 2: rel err vs oracle {err}"
    for b in (0, 15):
        target = dion_ref.polynomial_float64(x_cpu[b:b + 1].float(), dion_ref.GRAM_COEFFICIENTS,
                                             1.0, 1e-8)
        gpu_err = rel_fro(out_cpu[b:b + 1], target)
        oracle_err = rel_fro(ref[b:b + 1], target)
        assert gpu_err < 1.3 * oracle_err + 3e-3, f"block {b}: gpu {gpu_err} oracle {oracle_err}"


# ---- config 4: Llama-3-8B ------------------------------------------------------

LLAMA_LAYER = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
               ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]
# The step's Newton-Schulz runs at 32 layers: (blocks, selected rows, cols).
LLAMA_NS_RUNS = [(64, 1024, 4096), (64, 256, 4096), (64, 3584, 4096), (32, 1024, 14336)]


def test_config4_llama_layer_step() -> None:
    """One Llama-3-8B decoder layer (q/o 4096^2, k/v 1024 x 4096, gate/up
    14336 x 4096 with k = 3584, down 4096 x 14336 with k = 1024) through
    ``Dion.step`` with its four bucket runs queued and orthogonalized together,
    two steps, against the oracle on every block."""
    _say("config 4: one Llama-3-8B layer, 2 steps")
    g = torch.Generator(device=DEV).manual_seed(0)
    params = {name: nn.Parameter(_normal(g, rows, cols, std=0.02))
              for name, rows, cols in LLAMA_LAYER}
    opt = Dion([{"params": list(params.values()), ROUTE_KEY: "matrix", FRACTION_KEY: 0.25}],
               lr=LR, momentum=MU, muon_beta2=BETA2, weight_decay=WD)
    buckets = {"q/o": ["q", "o"], "k/v": ["k", "v"], "gate/up": ["gate", "up"], "down": ["down"]}
    ref = {}
    for bname, names in buckets.items():
        w = torch.stack([params[n].detach().cpu() for n in names])
        ref[bname] = (w, torch.zeros_like(w), torch.zeros(w.shape[0], w.shape[1], 1))
    for step in range(2):
        grads = {n: _normal(g, *params[n].shape, std=1e-3) for n in params}
        for n, p in params.items():
            p.grad = grads[n]
        before = {b: torch.stack([params[n].detach().cpu() for n in names])
                  for b, names in buckets.items()}
        opt.step()
        torch.cuda.synchronize()
        for bname, names in buckets.items():
            _, mom, var = ref[bname]
            w = before[bname].clone()
            rows = w.shape[1]
            grad = torch.stack([grads[n].cpu() for n in names])
            dion_ref.step_blocks(w, grad, mom, var, k=math.ceil(0.25 * rows), lr=LR, mu=MU,
                                 beta2=BETA2, weight_decay=WD, kind="gram")
            _check_run(f"step {step} {bname}", [params[n] for n in names], opt, before[bname], w,
                       mom, var, 1e-2)


def test_config4_llama3_8b_full_steps() -> None:
    """The whole Llama-3-8B step bench.py times (``bench.build_llama``: 32
    layers, Dion f = 0.25 on every linear, AdamW on the two 128256 x 4096
    embeddings with weight decay and on the 65 RMSNorm weights without), five
    steps with new gradients each. At every step: AdamW bit for bit against
    torch.optim.AdamW(fused=True) on twins of the same tensors (1.05 G
    elements, the embeddings' 128 k chunks per tensor included); every block's
    momentum and selection count; two sampled blocks per bucket against the
    oracle from the GPU's state before the step."""
    import bench

    _say("config 4: Llama-3-8B, all 32 layers, 5 steps")
    dev = torch.device(DEV)
    groups, n_params = bench.build_llama(torch, dev, bench.LLAMA, 0.25)
    assert n_params == 8_030_261_248
    embeds, norms, matrices = (grp["params"] for grp in groups)
    opt = Dion(groups, lr=LR, weight_decay=WD, momentum=MU, muon_beta2=BETA2,
               betas=(0.9, 0.95), eps=1e-8)
    twins = [nn.Parameter(p.detach().clone()) for p in embeds + norms]
    torch_opt = torch.optim.AdamW(
        [{"params": twins[:2]}, {"params": twins[2:], "weight_decay": 0.0}],
        lr=LR, betas=(0.9, 0.95), weight_decay=WD, eps=1e-8, fused=True)
    per_layer = len(LLAMA_LAYER)
    by_name = {name: matrices[i::per_layer] for i, (name, _, _) in enumerate(LLAMA_LAYER)}
    buckets = {"q/o": [p for pair in zip(by_name["q"], by_name["o"]) for p in pair],
               "k/v": [p for pair in zip(by_name["k"], by_name["v"]) for p in pair],
               "gate/up": [p for pair in zip(by_name["gate"], by_name["up"]) for p in pair],
               "down": by_name["down"]}
    g = torch.Generator(device=DEV).manual_seed(4)
    try:
        for step in range(5):
            for p in matrices + embeds + norms:
                p.grad.normal_(0.0, 1e-3, generator=g)
            for p, t in zip(embeds + norms, twins):
                t.grad = p.grad.clone()
            samples = {b: _sample(len(ps), step) for b, ps in buckets.items()}
            before = {b: _state_before(opt, ps, samples[b]) for b, ps in buckets.items()}
            m_old = {b: [_momentum_of(opt, p) for p in ps] for b, ps in buckets.items()}
            opt.step()
            torch_opt.step()
            torch.cuda.synchronize()
            _say(f"config 4: step {step} done, checking")
            for p, t in zip(embeds + norms, twins):
                assert torch.equal(p.detach(), t.detach()), f"step {step}: AdamW {tuple(p.shape)}"
            for bname, ps in buckets.items():
                k = math.ceil(0.25 * ps[0].shape[0])
                _check_every_block(f"step {step} {bname}", ps, opt, m_old[bname], k)
                _check_sampled(f"step {step} {bname}", ps, opt, samples[bname], before[bname], k)
            del m_old
    finally:
        del opt, torch_opt, twins, groups, embeds, norms, matrices, by_name, buckets
        _workspace.release()
        torch.cuda.empty_cache()


def test_config4_grouped_newton_schulz_at_bucket_shapes() -> None:
    """The Newton-Schulz call of a whole Llama-3-8B step: the four runs at their
    32-layer bucket sizes in one grouped call (the 24 launches bench.py times,
    256x256 tiles, gate/up dealt to the XCDs in runs of 32, Q X read as a
    [k, n] operand at k = 3584). Bit for bit equal to one call per run, and
    sampled blocks of every run against the oracle and the float64 polynomial."""
    _say("config 4: grouped Newton-Schulz at the bucket shapes")
    ortho = newton_schulz_fn(NewtonSchulz.GRAM)
    g = torch.Generator(device=DEV).manual_seed(40)
    stream = _lib.stream_handle(torch.device(DEV))
    xs, saved, outs, calls = [], [], [], []
    for i, (blocks, r, c) in enumerate(LLAMA_NS_RUNS):
        x = _normal(g, blocks, r, c)
        x = (x / torch.linalg.vector_norm(x, dim=(-2, -1), keepdim=True)).half()
        out = torch.empty(blocks, r, c, device=DEV, dtype=torch.bfloat16)
        xs.append(x)
        saved.append(x.clone())
        outs.append(out)
        calls.append(newton_schulz_call(ortho, blocks, r, c, x, None, out, f"cfg4_ns#{i}"))
    assert group_launches(calls) == 24
    try:
        run_newton_schulz_group(calls, stream)
        grouped = [o.clone() for o in outs]
        for x, s in zip(xs, saved):
            x.copy_(s)
        for call in calls:
            run_newton_schulz_call(call, stream)
        torch.cuda.synchronize()
        for (blocks, r, c), a, b in zip(LLAMA_NS_RUNS, grouped, outs):
            assert torch.equal(a, b), f"run {blocks} x {r} x {c}: grouped != separate calls"
        for (blocks, r, c), s, out in zip(LLAMA_NS_RUNS, saved, grouped):
            pick = [0, blocks - 1]
            x_cpu = s[pick].cpu()
            got = out[pick].cpu().float()
            ref = dion_ref._gram(x_cpu).bfloat16().float()
            err = rel_fro(got, ref)
            assert err < 1e-2, f"run {blocks} x {r} x {c}: rel err vs oracle {err}"
            if r == 3584:
                target = dion_ref.polynomial_float64(x_cpu[:1].float(), dion_ref.GRAM_COEFFICIENTS,
                                                     1.0, 1e-8)
                gpu_err, oracle_err = rel_fro(got[:1], target), rel_fro(ref[:1], target)
                assert gpu_err < 1.3 * oracle_err + 3e-3, f"gate/up: {gpu_err} vs {oracle_err}"
    finally:
        _workspace.release()


# ---- config 3: GPT-2 small -----------------------------------------------------

GPT2_MATRICES = [("qkv", 2304, 768), ("proj", 768, 768), ("fc", 3072, 768), ("fc2", 768, 3072)]


def test_config3_gpt2_small_step() -> None:
    """GPT-2 small (124 M parameters): 12 layers of qkv, proj, fc, fc2 on Dion
    with every row updated (768-wide sides), AdamW on wte 50257 x 768, wpe,
    LayerNorms and biases. Ten steps: every block's momentum, two sampled
    blocks per bucket against the oracle, AdamW bit for bit against
    torch.optim.AdamW(fused=True) at every step."""
    _say("config 3: GPT-2 small, 10 steps")
    g = torch.Generator(device=DEV).manual_seed(0)
    mats = {name: [nn.Parameter(_normal(g, rows, cols, std=0.02)) for _ in range(12)]
            for name, rows, cols in GPT2_MATRICES}
    embeds = [nn.Parameter(_normal(g, 50257, 768, std=0.02)),
              nn.Parameter(_normal(g, 1024, 768, std=0.02))]
    vectors = [nn.Parameter(_normal(g, n, std=0.02))
               for n in [2304, 768, 3072, 768, 768, 768, 768, 768] * 12 + [768, 768]]
    opt = Dion([{"params": [p for ps in mats.values() for p in ps], ROUTE_KEY: "matrix",
                 FRACTION_KEY: 1.0},
                {"params": embeds, ROUTE_KEY: "adamw"},
                {"params": vectors, ROUTE_KEY: "adamw", "weight_decay": 0.0}],
               lr=LR, momentum=MU, muon_beta2=BETA2, betas=(0.9, 0.95), weight_decay=WD)
    twins = [nn.Parameter(p.detach().clone()) for p in embeds + vectors]
    torch_opt = torch.optim.AdamW(
        [{"params": twins[:2]}, {"params": twins[2:], "weight_decay": 0.0}],
        lr=LR, betas=(0.9, 0.95), weight_decay=WD, eps=1e-8, fused=True)
    for step in range(10):
        for ps in mats.values():
            for p in ps:
                p.grad = _normal(g, *p.shape, std=1e-3)
        for p, t in zip(embeds + vectors, twins):
            p.grad = _normal(g, *p.shape, std=1e-3)
            t.grad = p.grad.clone()
        sample = _sample(12, step)
        before = {name: _state_before(opt, ps, sample) for name, ps in mats.items()}
        m_old = {name: [_momentum_of(opt, p) for p in ps] for name, ps in mats.items()}
        opt.step()
        torch_opt.step()
        torch.cuda.synchronize()
        for p, t in zip(embeds + vectors, twins):
            assert torch.equal(p.detach(), t.detach()), f"step {step}: AdamW {tuple(p.shape)}"
        for name, ps in mats.items():
            _check_every_block(f"step {step} {name}", ps, opt, m_old[name], ps[0].shape[0])
            _check_sampled(f"step {step} {name}", ps, opt, sample, before[name],
                           k=ps[0].shape[0])


# ---- config 5: MoE expert stack ---------------------------------------------------

def _experts(g: torch.Generator) -> list[nn.Parameter]:
    experts = []
    for _ in range(64):
        experts += [nn.Parameter(_normal(g, 1408, 2048, std=0.02)),
                    nn.Parameter(_normal(g, 1408, 2048, std=0.02)),
                    nn.Parameter(_normal(g, 2048, 1408, std=0.02))]
    return experts


def test_config5a_moe_dion_with_gpu_ema() -> None:
    """64 experts (gate/up 1408 x 2048 with k = 352, down 2048 x 1408 with k =
    512), Dion f = 0.25, Student-t(3) gradients, GPU EMA 0.9999 every step
    (a copy at step 1, then the lerp fused into the apply pass). Ten steps:
    every block's momentum and selection count, two sampled blocks per bucket
    against the oracle, and every shadow bit for bit against
    torch._foreach_lerp_ of the new weights."""
    _say("config 5a: MoE Dion + GPU EMA, 10 steps")
    g = torch.Generator(device=DEV).manual_seed(0)
    experts = _experts(g)
    opt = Dion([{"params": experts, ROUTE_KEY: "matrix", FRACTION_KEY: 0.25}], lr=LR,
               momentum=MU, muon_beta2=BETA2, weight_decay=WD,
               ema=EMAConfig(decay=0.9999, update_every_n_steps=1))
    buckets = {"gate/up": [p for i, p in enumerate(experts) if i % 3 != 2],
               "down": experts[2::3]}
    shadows = None
    for step in range(10):
        for p in experts:
            p.grad = _student_t(g, *p.shape)
        samples = {b: _sample(len(ps), step) for b, ps in buckets.items()}
        before = {b: _state_before(opt, ps, samples[b]) for b, ps in buckets.items()}
        m_old = {b: [_momentum_of(opt, p) for p in ps] for b, ps in buckets.items()}
        opt.step()
        opt.ema.flush_pending_updates()
        torch.cuda.synchronize()
        new_w = [p.detach().clone() for p in experts]
        if shadows is None:
            shadows = new_w
        else:
            torch._foreach_lerp_(shadows, new_w, 1.0 - 0.9999)
        for i, (p, s) in enumerate(zip(experts, shadows)):
            assert torch.equal(opt.state[p]["ema_shadow"], s), f"step {step}: shadow {i}"
        for bname, ps in buckets.items():
            k = math.ceil(0.25 * ps[0].shape[0])
            _check_every_block(f"step {step} {bname}", ps, opt, m_old[bname], k)
            _check_sampled(f"step {step} {bname}", ps, opt, samples[bname], before[bname], k)


def test_config5b_moe_muon_update() -> None:
    """The same 64 experts with MUON_UPDATE (KELLER_TRITON bfloat16 quintic,
    Nesterov, every row, no row normalization). Ten steps: momentum bit for
    bit on every expert, two sampled blocks per bucket against the oracle."""
    _say("config 5b: MoE MUON_UPDATE, 10 steps")
    g = torch.Generator(device=DEV).manual_seed(0)
    experts = _experts(g)
    opt = Dion([{"params": experts, ROUTE_KEY: "matrix", FRACTION_KEY: 1.0}], lr=LR,
               momentum=MU, muon_beta2=BETA2, weight_decay=WD, matrix_update=MUON_UPDATE)
    buckets = {"gate/up": [p for i, p in enumerate(experts) if i % 3 != 2],
               "down": experts[2::3]}
    for step in range(10):
        for p in experts:
            p.grad = _student_t(g, *p.shape)
        samples = {b: _sample(len(ps), step) for b, ps in buckets.items()}
        before = {b: _state_before(opt, ps, samples[b]) for b, ps in buckets.items()}
        m_old = {b: [_momentum_of(opt, p) for p in ps] for b, ps in buckets.items()}
        opt.step()
        torch.cuda.synchronize()
        for bname, ps in buckets.items():
            rows = ps[0].shape[0]
            _check_every_block(f"step {step} {bname}", ps, opt, m_old[bname], rows)
            _check_sampled(f"step {step} {bname}", ps, opt, samples[bname], before[bname],
                           rows, kind="keller_triton", normuon=False, nesterov=True)
