"""CPU restatement of the reference's Dion step (test infrastructure only).

Reference files: src/dionw/_matrix_step.py, _momentum_kernels.py, _gram.py,
_polar_express.py, _keller.py, _symmetric_kernels.py, _row_normalization.py,
_adamw.py, ema/_update.py. Products of 16-bit matrices are formed in float32
from the exact 16-bit values (a float16 x float16 product is exact in float32)
and rounded once to the storage dtype, as the reference's kernels store them.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Final

import numpy as np
import torch
from torch import Tensor

# ---- coefficient tables (the reference's, restated) ---------------------------

# _gram.py:26-38: Polar Express rows with the Gram safety factor 1.05 folded in.
_GRAM_RAW: Final = (
    (8.28721201814563, -23.595886519098837, 17.300387312530933),
    (4.107059111542203, -2.9478499167379106, 0.5448431082926601),
    (3.9486908534822946, -2.908902115962949, 0.5518191394370137),
    (3.3184196573706015, -2.488488024314874, 0.51004894012372),
    (2.300652019954817, -1.6689039845747493, 0.4188073119525673),
)
GRAM_COEFFICIENTS: Final = tuple((a / 1.05, b / 1.05**3, c / 1.05**5) for a, b, c in _GRAM_RAW)
GRAM_RESTART_ITERATION: Final = 2
# _polar_express.py:28-36.
POLAR_EXPRESS_COEFFICIENTS: Final = (
    (8.156554524902461, -22.48329292557795, 15.878769915207462),
    (4.042929935166739, -2.808917465908714, 0.5000178451051316),
    (3.8916678022926607, -2.772484153217685, 0.5060648178503393),
    (3.285753657755655, -2.3681294933425376, 0.46449024233003106),
    (2.3465413258596377, -1.7097828382687081, 0.42323551169305323),
)
POLAR_EXPRESS_NORM_SAFETY: Final = 1.02
# _keller.py:20-24.
KELLER_COEFFICIENTS: Final = ((3.4445, -4.7750, 2.0315),) * 5
KELLER_NORM_SAFETY: Final = 1.0

ADAMW_UPDATE_RMS: Final = 0.2          # _matrix_step.py:41
NEWTON_SCHULZ_EPS: Final = 1e-8        # _matrix_step.py:43
NORMALIZATION_EPS: Final = 1e-8        # _row_normalization.py:15


# ---- momentum passes (_momentum_kernels.py:40-77) -----------------------------

def row_l1_scores(m: np.ndarray) -> np.ndarray:
    """Row l1 norms of float32 ``m`` [rows, cols] in the kernel's fixed order.

    Follows the reduction of _momentum_kernels.py:44-55 (per-thread partial
    sums over column chunks, then a tree) in the order the HIP kernel fixes:
    thread t of 256 sums its float4 chunks ``t, t + 256, ...`` component-wise in
    column order and combines ``(x + y) + (z + w)``; within each of the four
    waves (threads 64w .. 64w + 63) lanes combine pairwise (i, i + 32),
    (i, i + 16), ..., (i, i + 1); the wave sums combine as (w0 + w1) + (w2 + w3).
    For cols % 4 != 0 thread t sums the single elements ``t, t + 256, ...``.
    """
    m = np.ascontiguousarray(m, dtype=np.float32)
    rows, cols = m.shape
    a = np.abs(m)
    threads = 256
    if cols % 4 == 0:
        n4 = cols // 4
        steps = -(-n4 // threads)
        padded = np.zeros((rows, steps * threads * 4), np.float32)
        padded[:, :cols] = a
        chunks = padded.reshape(rows, steps, threads, 4)
        part = np.zeros((rows, threads, 4), np.float32)
        for j in range(steps):
            part = part + chunks[:, j]
        lanes = (part[..., 0] + part[..., 1]) + (part[..., 2] + part[..., 3])
    else:
        steps = -(-cols // threads)
        padded = np.zeros((rows, steps * threads), np.float32)
        padded[:, :cols] = a
        chunks = padded.reshape(rows, steps, threads)
        lanes = np.zeros((rows, threads), np.float32)
        for j in range(steps):
            lanes = lanes + chunks[:, j]
    lanes = lanes.reshape(rows, 4, 64)
    off = 32
    while off >= 1:
        lanes = lanes[..., :off] + lanes[..., off : 2 * off]
        off //= 2
    w = lanes[..., 0]
    return ((w[:, 0] + w[:, 1]) + (w[:, 2] + w[:, 3])).astype(np.float32)


def topk_rows(scores: np.ndarray, k: int) -> np.ndarray:
    """The ``k`` largest scores' row indices, ascending; ties take lower rows.

    torch.topk(sorted=False) (_matrix_step.py:172-174) returns an unordered
    set; this fixes the tie rule the HIP kernel uses.
    """
    order = np.lexsort((np.arange(scores.shape[0]), -scores.astype(np.float64)))
    return np.sort(order[:k])


# ---- Newton-Schulz (_gram.py, _polar_express.py, _symmetric_kernels.py) -------

def _mm(a: Tensor, b: Tensor) -> Tensor:
    return torch.matmul(a.float(), b.float())


def ns_line_1(x: Tensor) -> Tensor:
    """``x x^T`` stored in x's dtype (_symmetric_kernels.py:81-144), exactly
    symmetric (the mirrored store)."""
    g = _mm(x, x.mT)
    g = torch.triu(g) + torch.triu(g, 1).mT
    return g.to(x.dtype)


def ns_line_2(a: Tensor, alpha: float, beta: float) -> Tensor:
    """``alpha a a^T + beta a`` for symmetric ``a`` (_symmetric_kernels.py:147-218)."""
    acc = _mm(a, a.mT) * alpha + a.float() * beta
    acc = torch.triu(acc) + torch.triu(acc, 1).mT
    return acc.to(a.dtype)


def _baddbmm(c: Tensor, a: Tensor, b: Tensor, beta: float) -> Tensor:
    """``beta c + a b`` in float32, stored in c's dtype (torch.baddbmm)."""
    return (_mm(a, b) + beta * c.float()).to(c.dtype)


def _gram(x: Tensor, restart: int | None = GRAM_RESTART_ITERATION) -> Tensor:
    """_gram.py:50-69 on wide float16 ``x`` [N, r, c]. ``restart=None`` never
    re-forms the Gram matrix from the iterate (a variant for tests that show
    what the restart buys)."""
    gram = ns_line_1(x)
    eye = torch.eye(x.size(-2), dtype=torch.float32).expand(gram.shape)
    q = None
    last = len(GRAM_COEFFICIENTS) - 1
    for i, (a, b, c) in enumerate(GRAM_COEFFICIENTS):
        if i == restart:
            x = _mm(q, x).to(x.dtype)
            gram = ns_line_1(x)
        z = ns_line_2(gram, c, b)
        if i in (0, restart):
            q = (z.float() + a * eye).to(x.dtype)
        else:
            q = _baddbmm(q, q, z, a)
        if i < last and i + 1 != restart:
            rz = _baddbmm(gram, gram, z, a)
            gram = _baddbmm(rz, z, rz, a)
    return _mm(q, x).to(x.dtype)


def _standard(x: Tensor) -> Tensor:
    """_gram.py:41-47: the standard iteration on square float16 blocks."""
    for a, b, c in GRAM_COEFFICIENTS:
        poly = ns_line_2(ns_line_1(x), c, b)
        x = _baddbmm(x, poly, x, a)
    return x


def gram_polar_express(matrix: Tensor, epsilon: float,
                       restart: int | None = GRAM_RESTART_ITERATION) -> Tensor:
    """_gram.py:72-89: Gram Newton-Schulz of a [N, rows, cols] batch, bf16 out."""
    tall = matrix.size(-2) > matrix.size(-1)
    x = matrix.mT if tall else matrix
    x = x.float()
    norm = torch.linalg.vector_norm(x, dim=(-2, -1), keepdim=True)
    x = (x / (norm + epsilon)).half().contiguous()
    x = _gram(x, restart) if x.size(-1) > x.size(-2) else _standard(x)
    return (x.mT if tall else x).bfloat16()


def _bf16_normalized(x: Tensor, epsilon: float, norm_safety: float) -> Tensor:
    """``x / (x.norm() * safety + eps)`` of bfloat16 ``x`` as the compiled
    reference evaluates it (_polar_express.py:57-58, 89-92): the norm is a
    float32 sum of the bf16 values stored as a bf16 tensor; the scaling and the
    division run in float32 and round once to bfloat16."""
    xf = x.float()
    norm = torch.linalg.vector_norm(xf, dim=(-2, -1), keepdim=True).bfloat16().float()
    return (xf / (norm * norm_safety + epsilon)).bfloat16()


def quintic(
    matrix: Tensor, epsilon: float, coefficients: tuple, norm_safety: float
) -> Tensor:
    """quintic_triton (_polar_express.py:74-104) in bfloat16: each line's product
    and elementwise terms from one float32 accumulation, rounded once."""
    tall = matrix.size(-2) > matrix.size(-1)
    x = matrix.to(torch.bfloat16)
    if tall:
        x = x.mT
    x = _bf16_normalized(x, epsilon, norm_safety).contiguous()
    for a, b, c in coefficients:
        poly = ns_line_2(ns_line_1(x), c, b)
        x = _baddbmm(x, poly, x, a)
    return x.mT if tall else x


def quintic_cublas(
    matrix: Tensor, epsilon: float, coefficients: tuple, norm_safety: float
) -> Tensor:
    """quintic_cublas (_polar_express.py:43-71) in bfloat16: every product is
    rounded to bfloat16 on its own (cuBLAS), and the elementwise terms
    ``b A + c (A A)`` and ``a x + (...)`` combine those bf16 products in float32
    with one rounding each (inductor fuses them). A tall block multiplies from
    the right (``x^T x``, ``x P``), a wide or square one from the left."""
    x = _bf16_normalized(matrix.to(torch.bfloat16), epsilon, norm_safety)
    tall = matrix.size(-2) > matrix.size(-1)
    for a, b, c in coefficients:
        gram = (_mm(x.mT, x) if tall else _mm(x, x.mT)).bfloat16()
        gram2 = _mm(gram, gram).bfloat16()
        poly = (b * gram.float() + c * gram2.float()).bfloat16()
        product = (_mm(x, poly) if tall else _mm(poly, x)).bfloat16()
        x = (a * x.float() + product.float()).bfloat16()
    return x


def polar_express(matrix: Tensor, epsilon: float) -> Tensor:
    """POLAR_EXPRESS (_polar_express.py:107-112): the cuBLAS quintic."""
    return quintic_cublas(matrix, epsilon, POLAR_EXPRESS_COEFFICIENTS, POLAR_EXPRESS_NORM_SAFETY)


def polar_express_triton(matrix: Tensor, epsilon: float) -> Tensor:
    """POLAR_EXPRESS_TRITON (_polar_express.py:115-120)."""
    return quintic(matrix, epsilon, POLAR_EXPRESS_COEFFICIENTS, POLAR_EXPRESS_NORM_SAFETY)


def keller(matrix: Tensor, epsilon: float) -> Tensor:
    """KELLER (_keller.py:25-28): the cuBLAS quintic."""
    return quintic_cublas(matrix, epsilon, KELLER_COEFFICIENTS, KELLER_NORM_SAFETY)


def keller_triton(matrix: Tensor, epsilon: float) -> Tensor:
    """KELLER_TRITON (_keller.py:31-34)."""
    return quintic(matrix, epsilon, KELLER_COEFFICIENTS, KELLER_NORM_SAFETY)


ORTHOGONALIZE = {
    "gram": gram_polar_express,
    "polar_express": polar_express,
    "polar_express_triton": polar_express_triton,
    "keller": keller,
    "keller_triton": keller_triton,
}


def polynomial_float64(x: Tensor, coefficients: tuple, norm_safety: float, epsilon: float = 1e-7) -> Tensor:
    """The Newton-Schulz polynomials of wide ``x`` evaluated in float64, no
    rounding (bench/precision.py:103-117): what every method approximates."""
    x = x.double()
    x = x / (x.norm(dim=(-2, -1), keepdim=True) * norm_safety + epsilon)
    for a, b, c in coefficients:
        g = x @ x.mT
        x = a * x + (b * g + c * g @ g) @ x
    return x


def exact_polar(x: Tensor) -> Tensor:
    """The exact polar factor U V^T by float64 SVD (tests/test_newton_schulz.py:41-43)."""
    u, _, vh = torch.linalg.svd(x.double(), full_matrices=False)
    return u @ vh


# ---- NorMuon and the step (_row_normalization.py, _matrix_step.py) ------------

def normalize_rows(update: Tensor, variance: Tensor, beta2: float, step: Tensor) -> tuple[Tensor, Tensor]:
    """_row_normalization.py:41-60 in float32 on the CPU."""
    u = update.float()
    norm = torch.linalg.vector_norm(u, dim=(-2, -1), keepdim=True)
    variance = torch.lerp(variance, u.square().mean(-1, keepdim=True), 1 - beta2)
    normalized = u / (variance.sqrt() + NORMALIZATION_EPS)
    new_norm = torch.linalg.vector_norm(normalized, dim=(-2, -1), keepdim=True)
    restore = norm / new_norm.clamp_min(NORMALIZATION_EPS)
    return normalized * (restore * step), variance


def step_size(rows: int, cols: int, k: int, lr: float) -> float:
    """_matrix_step.py:147-159."""
    return lr * ADAMW_UPDATE_RMS * math.sqrt(max(rows, cols)) * math.sqrt(min(rows, cols) / min(k, cols))


@dataclass
class RunResult:
    """What one oracle run step produced (for parity checks)."""

    index: np.ndarray | None      # [blocks, k] selected rows, ascending
    scores: np.ndarray | None     # [blocks, rows]
    orthogonal: Tensor            # [blocks, k, cols] bf16
    update: Tensor                # [blocks, k, cols] float32 (signed step included)


def step_blocks(
    weights: Tensor,
    grads: Tensor,
    momentum: Tensor,
    variance: Tensor,
    *,
    k: int,
    lr: float,
    mu: float,
    beta2: float,
    weight_decay: float,
    kind: str = "gram",
    normuon: bool = True,
    nesterov: bool = False,
    orthogonalize=None,
) -> RunResult:
    """One Dion step of a run of blocks, in place on CPU float32 tensors.

    ``weights``, ``grads``, ``momentum``: [blocks, rows, cols]; ``variance``:
    [blocks, rows, 1]. Follows step_run (_matrix_step.py:104-121): selected
    path (:162-199) when k < rows, full path (:202-251) otherwise, finish
    (_row_normalization.py:18-38) and _apply (:274-311).
    """
    blocks, rows, cols = (int(d) for d in weights.shape)
    step = torch.tensor(-step_size(rows, cols, k, lr), dtype=torch.float32)
    ortho = orthogonalize or ORTHOGONALIZE[kind]
    index = scores_out = None
    if k < rows:
        momentum += grads
        scores_out = np.stack([row_l1_scores(momentum[b].numpy()) for b in range(blocks)])
        index = np.stack([topk_rows(scores_out[b], k) for b in range(blocks)])
        idx = torch.from_numpy(index).long()
        gather = idx[:, :, None].expand(-1, -1, cols)
        selected = torch.gather(momentum, 1, gather)
        momentum.scatter_(1, gather, selected * mu)
        current = selected
        var_sel = torch.gather(variance, 1, idx[:, :, None])
    else:
        momentum += grads
        if nesterov:
            momentum.mul_(mu)
            current = momentum + grads
        else:
            current = momentum.clone()
            momentum.mul_(mu)
        var_sel = variance
    orthogonal = ortho(current, NEWTON_SCHULZ_EPS)
    if normuon:
        update, new_var = normalize_rows(orthogonal, var_sel, beta2, step)
        if index is None:
            variance.copy_(new_var)
        else:
            variance.scatter_(1, idx[:, :, None], new_var)
    else:
        update = orthogonal.float() * step
    if weight_decay > 0.0:
        weights.mul_(1.0 - lr * weight_decay)
    if index is None:
        weights.add_(update)
    else:
        weights.scatter_add_(1, gather, update)
    return RunResult(index, scores_out, orthogonal, update)


# ---- AdamW (_adamw.py:25-61 -> ATen fused AdamW) -------------------------------

def adamw(
    param: np.ndarray,
    grad: np.ndarray,
    exp_avg: np.ndarray,
    exp_avg_sq: np.ndarray,
    step: float,
    *,
    lr: float,
    beta1: float,
    beta2: float,
    weight_decay: float,
    eps: float,
) -> None:
    """One AdamW step in place, with ATen's fused AdamW promotions.

    Moments and weight decay in float64 rounded to float32; bias corrections
    in float64 handed over as float32; step size and denominator float32
    (torch/include/ATen/native/hip/fused_adam_utils.cuh, adam_math).
    ``step`` is the already incremented counter.
    """
    f32, f64 = np.float32, np.float64
    bc1 = f32(1 - beta1 ** float(step))
    bc2_sqrt = f32(math.sqrt(1 - beta2 ** float(step)))
    p = param.astype(f64)
    if weight_decay != 0:
        p = (p - lr * weight_decay * p).astype(f32)
    else:
        p = p.astype(f32)
    g = grad.astype(f64)
    m = (beta1 * exp_avg.astype(f64) + (1 - beta1) * g).astype(f32)
    v = (beta2 * exp_avg_sq.astype(f64) + (1 - beta2) * g * g).astype(f32)
    step_size_f = f32(lr / f64(bc1))
    denom = ((np.sqrt(v) / bc2_sqrt).astype(f64) + eps).astype(f32)
    p = p - (step_size_f * m) / denom
    param[...] = p
    exp_avg[...] = m
    exp_avg_sq[...] = v


# ---- EMA (ema/_update.py:17-29, ATen Lerp.h) -----------------------------------

def ema_lerp(shadow: np.ndarray, source: np.ndarray, decay: float) -> np.ndarray:
    """``lerp(shadow, source, 1 - decay)`` in float32 with ATen's two branches."""
    w = np.float32(1.0 - decay)
    s = shadow.astype(np.float32)
    p = source.astype(np.float32)
    if abs(w) < 0.5:
        return s + w * (p - s)
    return p - (p - s) * (np.float32(1.0) - w)
