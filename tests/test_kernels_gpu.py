"""HIP kernels against the CPU oracle and torch, through the C ABI (GPU).

Each test names its case in the assertion message. Bars: bit-exact for the
momentum add, the l1 scores (fixed reduction order), the row index sets, the
momentum decay, AdamW (vs torch._fused_adamw_) and the EMA (vs
torch._foreach_lerp_); rounding-derived tolerances for the 16-bit products.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from dionw_amd import _kernels, _lib, _workspace
from dionw_amd.newton_schulz import NewtonSchulz, newton_schulz_fn
from oracle import dion_ref
from tests.conftest import rel_fro

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


@pytest.mark.parametrize(("rows", "cols"), [(37, 3000), (64, 4096), (5, 1408), (17, 1001), (3, 6)])
def test_accumulate_scores_bit_exact(rows: int, cols: int) -> None:
    g = _gen(0)
    grad = torch.randn(rows, cols, generator=g)
    mom = torch.randn(rows, cols, generator=g)
    expected_m = mom + grad
    expected_scores = dion_ref.row_l1_scores(expected_m.numpy())
    grad_d, mom_d = grad.to(DEV), mom.to(DEV)
    scores = torch.empty(rows, device=DEV)
    _kernels.accumulate_row_l1(grad_d, mom_d, scores, cols)
    torch.cuda.synchronize()
    assert torch.equal(mom_d.cpu(), expected_m), f"M + G differs ({rows}x{cols})"
    got = scores.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), expected_scores.view(np.uint32)), (
        f"l1 scores not bit-exact ({rows}x{cols}), max diff {np.abs(got - expected_scores).max()}"
    )
    brute = np.abs(expected_m.double().numpy()).sum(-1)
    np.testing.assert_allclose(got, brute, rtol=1e-5)


def _select(scores: torch.Tensor, rowsq: torch.Tensor, k: int, *, elem: int = _lib.F16,
            safety: float = 1.0):
    blocks, rows = scores.shape
    idx = torch.empty(blocks, k, dtype=torch.int32, device=DEV)
    slot = torch.empty(blocks, rows, dtype=torch.int32, device=DEV)
    den = torch.empty(blocks, device=DEV)
    _lib.call("dionw_select_rows", scores.data_ptr(), rowsq.data_ptr(), blocks, rows, k, safety,
              1e-8, idx.data_ptr(), slot.data_ptr(), den.data_ptr(), elem,
              _lib.stream_handle())
    torch.cuda.synchronize()
    return idx.cpu().numpy(), slot.cpu().numpy(), den.cpu()


@pytest.mark.parametrize(("blocks", "rows", "k"), [(3, 1000, 250), (2, 14336, 3584), (4, 37, 37),
                                                   (1, 5, 1), (2, 4096, 1024)])
def test_select_rows_exact(blocks: int, rows: int, k: int) -> None:
    g = _gen(1)
    scores = torch.rand(blocks, rows, generator=g)
    scores[0, : rows // 3] = scores[0, rows // 3]  # a block full of ties
    rowsq = torch.rand(blocks, rows, generator=g)
    idx, slot, den = _select(scores.to(DEV), rowsq.to(DEV), k)
    for b in range(blocks):
        expected = dion_ref.topk_rows(scores[b].numpy(), k)
        assert np.array_equal(idx[b], expected), f"block {b}: index set differs ({rows}, {k})"
        inverse = np.full(rows, -1)
        inverse[expected] = np.arange(k)
        assert np.array_equal(slot[b], inverse), f"block {b}: slot map differs"
        ref_den = float(np.sqrt(rowsq[b].double().numpy()[expected].sum())) + 1e-8
        assert abs(float(den[b]) - ref_den) <= 1e-5 * ref_den


def test_select_rows_all_zero_scores() -> None:
    """Zero gradients leave every score at 0: the first k rows are taken."""
    scores = torch.zeros(2, 64, device=DEV)
    idx, _, _ = _select(scores, torch.zeros_like(scores), 16)
    assert np.array_equal(idx, np.tile(np.arange(16), (2, 1)))


@pytest.mark.parametrize("nesterov", [False, True])
def test_accumulate_copy_decay(nesterov: bool) -> None:
    g = _gen(2)
    grad, mom = torch.randn(5001, generator=g), torch.randn(5001, generator=g)
    s = mom + grad
    decayed = s * 0.95
    expected_out = grad + decayed if nesterov else s
    grad_d, mom_d = grad.to(DEV), mom.to(DEV)
    out = torch.empty(5001, device=DEV)
    _kernels.accumulate_copy_decay(grad_d, mom_d, out, 0.95, nesterov=nesterov)
    torch.cuda.synchronize()
    assert torch.equal(mom_d.cpu(), decayed), "decayed momentum not bit-exact"
    assert torch.equal(out.cpu(), expected_out), "Newton-Schulz input not bit-exact"


def _round8(n: int) -> int:
    return (n + 7) // 8 * 8


@pytest.mark.parametrize("elem", [0, 1], ids=["f16", "bf16"])
@pytest.mark.parametrize(("mode", "blocks", "rows", "cols", "k"), [
    ("selected", 3, 40, 4096, 12),    # float4 rows, padding rows past k
    ("selected", 2, 64, 1001, 16),    # ragged columns: scalar tail and padding columns
    ("every", 2, 37, 300, 37),        # every-row heavy ball
    ("nesterov", 2, 20, 14336, 20),   # wide rows
    ("every", 3, 9, 44, 9),           # short rows
])
def test_prepare_row_major_only(elem: int, mode: str, blocks: int, rows: int, cols: int,
                                k: int) -> None:
    """prepare_ns_input with the row-major output alone against the same call
    with both outputs: momentum and X bit-identical, the transpose exact, and X
    equal to fp16/bf16(U / den) restated on the CPU (IEEE division, one
    rounding)."""
    g = _gen(11)
    mom = torch.randn(blocks, rows, cols, generator=g)
    grad = torch.randn(blocks * rows, cols, generator=g)
    den = torch.rand(blocks, generator=g) * 50 + 1
    full = mode != "selected"
    idx = None
    if not full:
        idx = torch.stack([torch.randperm(rows, generator=g)[:k].sort().values
                           for _ in range(blocks)]).to(torch.int32)
    p_pad, j_pad = _round8(k) + 8, _round8(cols)
    mu, nesterov = 0.95, int(mode == "nesterov")
    dtype = torch.float16 if elem == 0 else torch.bfloat16
    grad_d, den_d = grad.to(DEV), den.to(DEV)
    idx_d = None if idx is None else idx.to(DEV)
    outs = []
    for both in (False, True):
        mom_d = mom.to(DEV)
        xr = torch.full((blocks, p_pad, j_pad), 7.0, device=DEV, dtype=dtype)  # padding overwritten
        xt = torch.empty(blocks, j_pad, p_pad, device=DEV, dtype=dtype) if both else None
        print(f"prepare {mode} {blocks}x{rows}x{cols} k={k} elem={elem} both={both}", flush=True)
        _lib.call("dionw_prepare_ns_input", _lib.ptr_array([grad_d]) if full else None,
                  1 if full else 0, mom_d.data_ptr(), None if idx_d is None else idx_d.data_ptr(),
                  den_d.data_ptr(), blocks, rows, cols, k, p_pad, j_pad, mu, nesterov, 1, elem,
                  xr.data_ptr(), None if xt is None else xt.data_ptr(), _lib.stream_handle())
        torch.cuda.synchronize()
        outs.append((mom_d.cpu(), xr.cpu(), None if xt is None else xt.cpu()))
    (m1, x1, _), (m2, x2, t2) = outs
    assert torch.equal(m1, m2), "decayed momentum differs between the two kernels"
    assert torch.equal(x1, x2), "row-major input differs between the two kernels"
    assert torch.equal(t2, x2.mT), "transposed output is not the transpose"
    # CPU restatement of U and X = U / den rounded once (bf16 input rounded first).
    if full:
        s = mom + grad.view(blocks, rows, cols)
        decayed = s * mu
        u = grad.view(blocks, rows, cols) + decayed if nesterov else s
        expected_m = decayed
    else:
        sel = torch.stack([mom[b, idx[b].long()] for b in range(blocks)])
        u = sel
        expected_m = mom.clone()
        for b in range(blocks):
            expected_m[b, idx[b].long()] = sel[b] * mu
    if elem == 1:
        u = u.to(torch.bfloat16).float()
    x = (u / den.view(-1, 1, 1)).to(dtype)
    expected_x = torch.zeros(blocks, p_pad, j_pad, dtype=dtype)
    expected_x[:, :k, :cols] = x
    assert torch.equal(m1, expected_m), "momentum differs from the restatement"
    assert torch.equal(x1, expected_x), "X differs from the restatement"


@pytest.mark.parametrize("x_dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("elem", [0, 1], ids=["f16", "bf16"])
@pytest.mark.parametrize(("blocks", "rows", "cols", "offset"),
                         [(3, 64, 256, 0), (2, 37, 300, 0), (2, 9, 1001, 0),
                          # 16-byte rows with a partial last tile and padding rows
                          (2, 100, 1032, 0), (1, 130, 4096, 0),
                          # 16-byte rows from an address 8 bytes past a 16-byte boundary
                          (2, 100, 1032, 4)])
def test_normalize_input_reads_16bit_inputs(x_dtype, elem: int, blocks: int, rows: int,
                                            cols: int, offset: int) -> None:
    """dionw_normalize_input on an fp16 / bf16 / fp32 input against
    full_sumsq + block_denom + prepare_ns_input on its float32 copy (vector and
    scalar paths): row sums, denominators and both outputs bit-identical."""
    g = _gen(12)
    n = blocks * rows * cols
    flat = (torch.randn(n + offset, generator=g) * 3).to(x_dtype).to(DEV)
    x = flat[offset:].view(blocks, rows, cols)
    src = x.float().contiguous()
    p_pad, j_pad = _round8(rows), _round8(cols)
    dtype = torch.float16 if elem == 0 else torch.bfloat16
    st = _lib.stream_handle()
    results = []
    for fused in (True, False):
        rowsq = torch.empty(blocks * rows, device=DEV)
        den = torch.empty(blocks, device=DEV)
        xr = torch.full((blocks, p_pad, j_pad), 5.0, device=DEV, dtype=dtype)
        xt = torch.full((blocks, j_pad, p_pad), 5.0, device=DEV, dtype=dtype)
        print(f"normalize {x_dtype} {blocks}x{rows}x{cols} elem={elem} fused={fused}", flush=True)
        if fused:
            _lib.call("dionw_normalize_input", x.data_ptr(), {torch.float16: 0, torch.bfloat16: 1,
                      torch.float32: 2}[x_dtype], blocks, rows, cols, 1.02, 1e-7,
                      rowsq.data_ptr(), den.data_ptr(), p_pad, j_pad, elem, xr.data_ptr(),
                      xt.data_ptr(), st)
        else:
            grads = _lib.ptr_array([src])
            _lib.call("dionw_full_sumsq", grads, 1, blocks * rows, cols, None, 0.0, 0,
                      rowsq.data_ptr(), elem, st)
            _lib.call("dionw_block_denom", rowsq.data_ptr(), blocks, rows, 1.02, 1e-7,
                      den.data_ptr(), elem, st)
            _lib.call("dionw_prepare_ns_input", grads, 1, None, None, den.data_ptr(), blocks,
                      rows, cols, rows, p_pad, j_pad, 0.0, 0, 0, elem, xr.data_ptr(),
                      xt.data_ptr(), st)
        torch.cuda.synchronize()
        results.append([t.cpu() for t in (rowsq, den, xr, xt)])
    for name, a, b in zip(("row sums", "den", "X", "X^T"), *results):
        assert torch.equal(a, b), f"{name} differs ({x_dtype}, {blocks}x{rows}x{cols})"


@pytest.mark.parametrize("kind", [NewtonSchulz.GRAM, NewtonSchulz.POLAR_EXPRESS,
                                  NewtonSchulz.KELLER])
@pytest.mark.parametrize("x_dtype", [torch.float16, torch.bfloat16])
def test_orthogonalize_16bit_input_equals_its_float32_copy(kind, x_dtype) -> None:
    """A 16-bit input is read as it is; its conversion to float32 is exact, so
    the result equals that of the float32 copy bit for bit."""
    g = _gen(13)
    x = torch.randn(3, 96, 200, generator=g).to(x_dtype).to(DEV)
    fn = newton_schulz_fn(kind)
    a, b = fn(x, 1e-7), fn(x.float(), 1e-7)
    torch.cuda.synchronize()
    assert torch.equal(a.cpu(), b.cpu()), f"{kind.value} {x_dtype}"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize(("batch", "m", "n", "k"), [(1, 64, 64, 64), (3, 100, 72, 136),
                                                    (2, 256, 512, 1024), (5, 352, 352, 2048),
                                                    # pipelined 128x128 tiles, 64-deep stages
                                                    (20, 1024, 1024, 512), (20, 1000, 1032, 512),
                                                    # pipelined 128x128 tiles, 32-deep stages
                                                    (20, 1024, 1024, 352),
                                                    # pipelined 256x256 tiles, 64- and 32-deep
                                                    (64, 1024, 1024, 512), (64, 1000, 1032, 352)])
def test_gemm_nt_matches_fp32(dtype: torch.dtype, batch: int, m: int, n: int, k: int) -> None:
    g = _gen(3)
    a = torch.randn(batch, m, k, generator=g).to(dtype)
    b = torch.randn(batch, n, k, generator=g).to(dtype)
    d = torch.randn(batch, m, n, generator=g).to(dtype)
    expected = (0.7 * (a.float() @ b.float().mT) - 1.3 * d.float()).to(dtype)
    out = torch.empty(batch, m, n, dtype=dtype, device=DEV)
    out_t = torch.empty(batch, n, m, dtype=dtype, device=DEV)
    _kernels.gemm_nt(a.to(DEV), b.to(DEV), d=d.to(DEV), alpha=0.7, beta=-1.3, out=out, out_t=out_t)
    torch.cuda.synchronize()
    tol = 2e-3 if dtype == torch.float16 else 1e-2
    err = rel_fro(out.cpu(), expected)
    assert err < tol, f"gemm {batch}x{m}x{n}x{k} {dtype}: rel err {err}"
    assert torch.equal(out_t.cpu(), out.cpu().mT), "transposed store differs"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape", [(3, 64, 256), (3, 128, 128), (96, 160), (2, 520, 1032)])
def test_symmetric_products(dtype: torch.dtype, shape: tuple[int, ...]) -> None:
    _check_symmetric(dtype, shape)


@pytest.mark.parametrize("shape", [(3, 64, 256), (2, 100, 70), (130, 37), (2, 520, 1032)])
def test_float32_symmetric_products(shape: tuple[int, ...]) -> None:
    """float32 ns_line_1 / ns_line_2 (the reference's "ieee" path for float32
    inputs, _symmetric_kernels.py:275, 311) on the fp32 MFMA: within float32
    rounding of float64 products, exactly symmetric, any size."""
    g = _gen(14)
    x = torch.randn(*shape, generator=g) / shape[-1] ** 0.5
    gram = _kernels.ns_line_1(x.to(DEV))
    torch.cuda.synchronize()
    assert gram.dtype == torch.float32
    ref = x.double() @ x.double().mT
    assert rel_fro(gram.cpu(), ref) < 1e-6, f"ns_line_1 fp32 {shape}"
    assert torch.equal(gram.cpu(), gram.cpu().mT), "ns_line_1 fp32 output not exactly symmetric"
    poly = _kernels.ns_line_2(gram, alpha=0.5, beta=-1.5)
    torch.cuda.synchronize()
    g64 = gram.cpu().double()
    ref2 = 0.5 * (g64 @ g64) - 1.5 * g64
    assert rel_fro(poly.cpu(), ref2) < 1e-6, f"ns_line_2 fp32 {shape}"
    assert torch.equal(poly.cpu(), poly.cpu().mT)


def test_float32_gemm_with_transposed_output_and_strides() -> None:
    """A float32 product of operands with padded row strides, an addend and a
    transposed second output, against float64."""
    g = _gen(15)
    a = torch.randn(2, 70, 50, generator=g)
    b = torch.randn(2, 90, 50, generator=g)
    d = torch.randn(2, 70, 90, generator=g)
    a_pad = torch.zeros(2, 70, 56)
    a_pad[..., :50] = a
    a_d = a_pad.to(DEV)[..., :50]
    out_t = torch.empty(2, 90, 70, device=DEV)
    out = _kernels.gemm_nt(a_d, b.to(DEV), d=d.to(DEV), alpha=0.7, beta=-1.3, out_t=out_t,
                           out=torch.empty(2, 70, 90, device=DEV))
    torch.cuda.synchronize()
    ref = 0.7 * (a.double() @ b.double().mT) - 1.3 * d.double()
    assert rel_fro(out.cpu(), ref) < 1e-6
    assert torch.equal(out_t.cpu(), out.cpu().mT)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_symmetric_products_pipelined(dtype: torch.dtype) -> None:
    """Batches large enough for the pipelined 256x256 kernel, ragged 1000 rows."""
    _check_symmetric(dtype, (40, 1024, 1024))
    _check_symmetric(dtype, (48, 1000, 1024))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_idle_waves_change_no_stored_element(dtype: torch.dtype) -> None:
    """The 256x256 kernel's waves skip their MFMAs where nothing they compute is
    stored: below the diagonal of a diagonal tile, and past a ragged side. The
    symmetric product of a symmetric matrix equals the full product bit for bit
    (1152 rows: 4.5 tiles), and a product with 1408 rows and 1920 columns equals
    the same rows and columns of its zero-padded 1536 x 2048 twin."""
    g = _gen(5)
    x = (torch.randn(48, 1152, 1152, generator=g) / 34).to(dtype)
    s = (x + x.mT).to(DEV)
    sym = _kernels.gemm_nt(s, s, d=s, alpha=0.5, beta=-1.5, symmetric=True)
    full = _kernels.gemm_nt(s, s, d=s, alpha=0.5, beta=-1.5, symmetric=False)
    torch.cuda.synchronize()
    assert torch.equal(sym, full), f"symmetric vs full product, 48 x 1152^2 {dtype}"
    a = (torch.randn(16, 1408, 1408, generator=g) / 38).to(dtype)
    b = (torch.randn(16, 1920, 1408, generator=g) / 38).to(dtype)
    a_pad = torch.zeros(16, 1536, 1408, dtype=dtype)
    b_pad = torch.zeros(16, 2048, 1408, dtype=dtype)
    a_pad[:, :1408], b_pad[:, :1920] = a, b
    ragged = _kernels.gemm_nt(a.to(DEV), b.to(DEV))
    padded = _kernels.gemm_nt(a_pad.to(DEV), b_pad.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(ragged, padded[:, :1408, :1920]), f"ragged 1408 x 1920 product {dtype}"


def _check_symmetric(dtype: torch.dtype, shape: tuple[int, ...]) -> None:
    g = _gen(4)
    x = (torch.randn(*shape, generator=g) / shape[-1] ** 0.5).to(dtype)
    gram = _kernels.ns_line_1(x.to(DEV))
    torch.cuda.synchronize()
    ref = dion_ref.ns_line_1(x)
    tol = 2e-3 if dtype == torch.float16 else 1e-2
    assert rel_fro(gram.cpu(), ref) < tol, f"ns_line_1 {shape} {dtype}"
    assert torch.equal(gram.cpu(), gram.cpu().mT), "ns_line_1 output not exactly symmetric"
    poly = _kernels.ns_line_2(gram, alpha=0.5, beta=-1.5)
    torch.cuda.synchronize()
    ref2 = dion_ref.ns_line_2(gram.cpu(), 0.5, -1.5)
    assert rel_fro(poly.cpu(), ref2) < tol, f"ns_line_2 {shape} {dtype}"
    assert torch.equal(poly.cpu(), poly.cpu().mT)


# Short sides that are multiples of 32 read the iterate directly in the left
# products; the others (40, 72, 104, 1400) read its transpose. Ragged ones pad;
# an odd multiple of 32 (288) next to a long side less than 32 longer stays
# unpadded.
NS_SHAPES = [(3, 64, 256), (3, 256, 64), (3, 128, 128), (2, 96, 160), (4, 256, 1024), (1, 352, 2048),
             (2, 30, 300), (2, 300, 30), (2, 40, 200), (2, 200, 40), (1, 72, 72), (2, 100, 520),
             (1, 288, 296), (1, 296, 288), (1, 288, 288),
             # Sides with a ragged last 256-row tile (MoE-Muon's 1408 = 5 x 256 + 128;
             # 1400, whose transpose is read), wide, tall and square.
             (1, 1408, 2048), (1, 2048, 1408), (1, 1400, 1600), (1, 1408, 1408)]

# Each kind's polynomials and norm safety (what its rounding is measured against).
POLYNOMIALS = {
    NewtonSchulz.GRAM: (dion_ref.GRAM_COEFFICIENTS, 1.0),
    NewtonSchulz.POLAR_EXPRESS: (dion_ref.POLAR_EXPRESS_COEFFICIENTS,
                                 dion_ref.POLAR_EXPRESS_NORM_SAFETY),
    NewtonSchulz.POLAR_EXPRESS_TRITON: (dion_ref.POLAR_EXPRESS_COEFFICIENTS,
                                        dion_ref.POLAR_EXPRESS_NORM_SAFETY),
    NewtonSchulz.KELLER: (dion_ref.KELLER_COEFFICIENTS, dion_ref.KELLER_NORM_SAFETY),
    NewtonSchulz.KELLER_TRITON: (dion_ref.KELLER_COEFFICIENTS, dion_ref.KELLER_NORM_SAFETY),
}


def polynomial_target(kind: NewtonSchulz, x: torch.Tensor) -> torch.Tensor:
    """The kind's polynomials in float64 on ``x`` (tall blocks in their wide
    orientation, returned in ``x``'s): what its rounding is measured against."""
    tall = x.shape[-2] > x.shape[-1]
    target = dion_ref.polynomial_float64(x.mT if tall else x, *POLYNOMIALS[kind])
    return target.mT if tall else target


@pytest.mark.parametrize("shape", NS_SHAPES)
@pytest.mark.parametrize("kind", list(NewtonSchulz))
def test_newton_schulz_matches_oracle(kind: NewtonSchulz, shape: tuple[int, ...]) -> None:
    """Every kind against its oracle, with bars derived from the oracle's own
    rounding error ``e`` (its distance to the same polynomials in float64):
    the HIP result rounds no worse (within ``1.3 e + 3e-3`` of the float64
    polynomials, the reference's own bar, test_newton_schulz.py:67-76), and lies
    within ``1.6 e + 3e-3`` of the oracle (the same rounding points in another
    accumulation order: about sqrt(2) e apart where the roundings are
    independent). ``e`` is 0.002-0.004 for Gram (0.016 near square, where the
    Gram matrix squares the condition number), 0.011-0.024 for the bf16
    quintics and up to 0.035 for the cuBLAS-rounded Polar Express."""
    g = _gen(5)
    x = torch.randn(*shape, generator=g)
    out = newton_schulz_fn(kind)(x.to(DEV), 1e-7)
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16 and out.shape == x.shape
    got = out.cpu().float()
    ref = dion_ref.ORTHOGONALIZE[kind.value](x, 1e-7).float()
    target = polynomial_target(kind, x)
    oracle_err = rel_fro(ref, target)
    gpu_err = rel_fro(got, target)
    assert gpu_err < 1.3 * oracle_err + 3e-3, (
        f"{kind.value} {shape}: {gpu_err} from the float64 polynomial, oracle {oracle_err}")
    diff = rel_fro(got, ref)
    assert diff < 1.6 * oracle_err + 3e-3, (
        f"{kind.value} {shape}: {diff} from the oracle (oracle rounding {oracle_err})")
    # Keller's quintic pushes singular values into about [0.7, 1.2], not onto 1.
    polar_bar = 0.3 if kind in (NewtonSchulz.KELLER, NewtonSchulz.KELLER_TRITON) else 0.2
    exact_err = rel_fro(got, dion_ref.exact_polar(x))
    assert exact_err < polar_bar, f"{kind.value} {shape}: {exact_err} from the exact polar factor"


@pytest.mark.parametrize(("cublas", "triton"), [
    (NewtonSchulz.POLAR_EXPRESS, NewtonSchulz.POLAR_EXPRESS_TRITON),
    (NewtonSchulz.KELLER, NewtonSchulz.KELLER_TRITON)])
@pytest.mark.parametrize("shape", [(2, 256, 1024), (2, 1024, 256)])
def test_quintic_variants_round_as_their_reference_twins(cublas, triton, shape) -> None:
    """The two quintic variants round at different points (_polar_express.py:
    43-104): each HIP kind is much closer to its own oracle than to the other
    variant's, so the products really are rounded where the variant says."""
    g = _gen(16)
    x = torch.randn(*shape, generator=g)
    for kind, other in ((cublas, triton), (triton, cublas)):
        out = newton_schulz_fn(kind)(x.to(DEV), 1e-8)
        torch.cuda.synchronize()
        same = rel_fro(out.cpu().float(), dion_ref.ORTHOGONALIZE[kind.value](x, 1e-8).float())
        cross = rel_fro(out.cpu().float(), dion_ref.ORTHOGONALIZE[other.value](x, 1e-8).float())
        assert same < 0.5 * cross, f"{kind.value} {shape}: own oracle {same}, other {cross}"


def test_bf16_norms_round_as_the_quintics() -> None:
    """With the bf16 norm element type the row sums of squares are of the
    bf16-rounded momentum and the denominator is bf16(sqrt(sum)) * safety + eps
    (_polar_express.py:57-58); the l1 scores are unchanged."""
    g = _gen(17)
    blocks, rows, cols, k = 2, 300, 512, 75
    grad = torch.randn(blocks * rows, cols, generator=g)
    mom = torch.randn(blocks * rows, cols, generator=g)
    st = _lib.stream_handle()
    out = {}
    for elem in (_lib.F16, _lib.BF16):
        m_d = mom.to(DEV)
        scores = torch.empty(blocks * rows, device=DEV)
        rowsq = torch.empty(blocks * rows, device=DEV)
        _lib.call("dionw_accumulate_scores", _lib.ptr_array([grad.to(DEV)]), 1, blocks * rows,
                  cols, m_d.data_ptr(), scores.data_ptr(), rowsq.data_ptr(), elem, st)
        idx, _, den = _select(scores.view(blocks, rows), rowsq.view(blocks, rows), k, elem=elem,
                              safety=1.02)
        out[elem] = (scores.cpu(), rowsq.cpu(), idx, den)
    assert torch.equal(out[_lib.F16][0], out[_lib.BF16][0]), "scores depend on the norm type"
    summed = (mom + grad)
    want_sq = summed.bfloat16().double().square().sum(-1)
    assert rel_fro(out[_lib.BF16][1], want_sq) < 1e-6
    want_sq32 = summed.double().square().sum(-1)
    assert rel_fro(out[_lib.F16][1], want_sq32) < 1e-6
    for b in range(blocks):
        rows_b = torch.from_numpy(out[_lib.BF16][2][b]).long()
        s = float(out[_lib.BF16][1].view(blocks, rows)[b, rows_b].double().sum())
        norm = float(torch.tensor(s ** 0.5, dtype=torch.float32).bfloat16().float())
        want_den = norm * 1.02 + 1e-8
        assert abs(float(out[_lib.BF16][3][b]) - want_den) <= 2e-6 * want_den, b


@pytest.mark.parametrize("shape", [(1, 256, 1024), (2, 1024, 4096)])
def test_gram_rounding_error_vs_float64_polynomial(shape: tuple[int, ...]) -> None:
    """Rounding error of the fp16 Gram iteration against the same polynomial in
    float64 (bench/precision.py method; the reference measures 0.003 on
    Gaussian 256 x 1024 input)."""
    g = _gen(6)
    x = torch.randn(*shape, generator=g)
    out = newton_schulz_fn(NewtonSchulz.GRAM)(x.to(DEV), 1e-7)
    torch.cuda.synchronize()
    target = dion_ref.polynomial_float64(x, dion_ref.GRAM_COEFFICIENTS, 1.0)
    err = rel_fro(out.cpu().float(), target)
    oracle_err = rel_fro(dion_ref.gram_polar_express(x, 1e-7).float(), target)
    assert err < 1.3 * oracle_err + 3e-3, f"{shape}: gpu {err} vs oracle {oracle_err}"
    assert err < 0.01


def test_adamw_bit_exact_vs_torch_fused() -> None:
    from dionw_amd._adamw import adamw_step, init_adamw_state

    g = _gen(7)
    shapes = [(1000,), (37, 61), (4096, 3), (1,), (70000,)]
    params = [torch.randn(*s, generator=g).to(DEV) for s in shapes]
    ref_params = [p.clone() for p in params]
    state: dict = {}
    for p in params:
        state[p] = {}
        init_adamw_state(p, state[p])
    ref_m = [torch.zeros_like(p) for p in params]
    ref_v = [torch.zeros_like(p) for p in params]
    ref_steps = [torch.zeros((), device=DEV) for _ in params]
    group = {"params": params, "lr": 3e-4, "betas": (0.9, 0.95), "weight_decay": 0.05, "eps": 1e-8}
    for it in range(4):
        grads = [torch.randn(*s, generator=g).to(DEV) * 1e-3 for s in shapes]
        for p, gr in zip(params, grads):
            p.grad = gr.clone()
        adamw_step(group, state)
        torch._foreach_add_(ref_steps, 1)
        torch._fused_adamw_(ref_params, grads, ref_m, ref_v, [], ref_steps, amsgrad=False,
                            lr=3e-4, beta1=0.9, beta2=0.95, weight_decay=0.05, eps=1e-8,
                            maximize=False, grad_scale=None, found_inf=None)
        torch.cuda.synchronize()
        for i, p in enumerate(params):
            assert torch.equal(p, ref_params[i]), f"step {it} tensor {i}: param not bit-exact"
            assert torch.equal(state[p]["exp_avg"], ref_m[i]), f"step {it} tensor {i}: exp_avg"
            assert torch.equal(state[p]["exp_avg_sq"], ref_v[i]), f"step {it} tensor {i}: exp_avg_sq"
            assert torch.equal(state[p]["adamw_step"], ref_steps[i])


@pytest.mark.parametrize("decay", [0.9999, 0.3, 0.5])
def test_ema_bit_exact_vs_torch_lerp(decay: float) -> None:
    from dionw_amd.ema._update import foreach_ema_copy_, foreach_ema_update_

    g = _gen(8)
    shapes = [(1000,), (37, 61), (70001,)]
    shadows = [torch.randn(*s, generator=g).to(DEV) for s in shapes]
    sources = [torch.randn(*s, generator=g).to(DEV) for s in shapes]
    ref = [s.clone() for s in shadows]
    foreach_ema_update_(shadows, sources, decay=decay)
    torch._foreach_lerp_(ref, sources, 1.0 - decay)
    torch.cuda.synchronize()
    for i in range(len(shapes)):
        assert torch.equal(shadows[i], ref[i]), f"lerp tensor {i} decay {decay}"
    constant = [s.clone() for s in sources]
    foreach_ema_update_(constant, sources, decay=decay)
    for c, s in zip(constant, sources):
        assert torch.equal(c, s), "a constant source must keep a bit-exact shadow"
    copies = [torch.empty_like(s) for s in sources]
    foreach_ema_copy_(copies, sources)
    for c, s in zip(copies, sources):
        assert torch.equal(c, s)


def test_workspace_is_reused() -> None:
    a = _workspace.buffer(torch.device(DEV), "t", (10,), torch.float32)
    b = _workspace.buffer(torch.device(DEV), "t", (5,), torch.float32)
    assert a.data_ptr() == b.data_ptr()
