"""Newton-Schulz orthogonalization of the matrix updates (``NewtonSchulz`` kinds on HIP kernels).

Reference: src/dionw/newton_schulz.py:30-68, the plugin boundary. Each kind
maps a ``[N, rows, cols]`` batch (any float dtype) and the epsilon added to its
Frobenius norm to the bfloat16 polar-factor approximations, five polynomial
steps each, on the MFMA kernels of ``libdionw_hip.so``:

- ``GRAM``: float16 Gram Newton-Schulz on ``X X^T`` with a restart at
  iteration 2 (wide blocks; tall ones are transposed, square ones run the
  standard Polar Express iteration), output bf16(fp16);
- ``POLAR_EXPRESS`` / ``POLAR_EXPRESS_TRITON``: the bfloat16 Polar Express
  quintic, input scaled by 1.02 times its norm;
- ``KELLER`` / ``KELLER_TRITON``: Keller Jordan's bfloat16 quintic.

The two variants of each quintic differ in where they round, and keep the
reference's difference (_polar_express.py:43-104): the ``_TRITON`` kinds round
each line once (``c A A + b A`` and ``a X + P X`` from float32 accumulators),
the others round the products ``A A`` and ``P X`` to bfloat16 before the
elementwise terms, as separate cuBLAS products do. Both run the same symmetric
MFMA products; a tall block is iterated in its wide orientation, whose products
are the transposes of the reference's right-hand ones.
"""

from __future__ import annotations

from collections.abc import Callable
from dataclasses import dataclass
from enum import Enum

import ctypes

import torch
from torch import Tensor

from dionw_amd import _lib, _workspace

__all__ = ["NewtonSchulz", "Orthogonalize", "HipOrthogonalize", "newton_schulz_fn"]

# Signature of an orthogonalization: a [N, rows, cols] batch and epsilon in, bf16 batch out.
Orthogonalize = Callable[[Tensor, float], Tensor]

# Library kinds (include/dionw_hip.h, dionw_newton_schulz).
_GRAM, _PE_TRITON, _KELLER_TRITON, _PE_CUBLAS, _KELLER_CUBLAS = 0, 1, 2, 3, 4
# Input types dionw_normalize_input reads as they are.
_INPUT_ELEMS = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}


class NewtonSchulz(Enum):
    """The Newton-Schulz iteration (and its rounding variant) that orthogonalizes an update."""

    POLAR_EXPRESS = "polar_express"
    POLAR_EXPRESS_TRITON = "polar_express_triton"
    GRAM = "gram"
    KELLER = "keller"
    KELLER_TRITON = "keller_triton"


def _round8(n: int) -> int:
    return (n + 7) // 8 * 8


# Whether an iterate whose short side is an odd multiple of 32 (at least 256)
# is padded with zero rows to the next multiple of 64.
PAD_SHORT_SIDE_TO_64 = True


def padded_sides(rows: int, cols: int) -> tuple[int, int]:
    """The padded extents ``(p_pad, j_pad)`` of a ``[rows, cols]`` block's
    prepared input: both sides rounded up to 8; a short side that is then an odd
    multiple of 32 (at least 256) grows by 32 more, so that the products whose
    depth is that side run 64-deep LDS stages (the padding rows are zero, which
    every polynomial here keeps exactly zero, and are never stored).

    The short side grows only while it stays no longer than the long side: the
    iteration runs in the orientation of the unpadded block (wide: short side
    first), and the library needs the first padded extent to be the shorter.
    """
    p_pad, j_pad = _round8(rows), _round8(cols)
    short, long = min(p_pad, j_pad), max(p_pad, j_pad)
    if PAD_SHORT_SIDE_TO_64 and short >= 256 and short % 64 == 32 and short + 32 <= long:
        if rows <= cols:
            p_pad += 32
        else:
            j_pad += 32
    return p_pad, j_pad


def prepared_orientations(rows: int, cols: int) -> tuple[bool, bool]:
    """Which prepared inputs the iteration on ``[rows, cols]`` blocks reads:
    (weight orientation, its transpose).

    The iterate is the wide orientation (the transpose of a tall block). The
    library reads the iterate's transpose only when the short side, rounded up
    to 8, is not a multiple of 32; otherwise its left products take the iterate
    itself as a ``[k, n]`` operand (``dionw_newton_schulz``).
    """
    tall = rows > cols
    other = min(padded_sides(rows, cols)) % 32 != 0
    return (other, True) if tall else (True, other)


def prepared_inputs(
    ortho: HipOrthogonalize, device: torch.device, blocks: int, rows: int, cols: int,
    name_xr: str, name_xt: str,
) -> tuple[Tensor | None, Tensor | None]:
    """Scratch buffers for the prepared inputs of ``[blocks, rows, cols]``: the
    weight orientation ``[blocks, round8(rows), round8(cols)]`` and its
    transpose, each None when the iteration does not read it."""
    p_pad, j_pad = padded_sides(rows, cols)
    want_xr, want_xt = prepared_orientations(rows, cols)
    xr = (_workspace.buffer(device, name_xr, (blocks, p_pad, j_pad), ortho.dtype)
          if want_xr else None)
    xt = (_workspace.buffer(device, name_xt, (blocks, j_pad, p_pad), ortho.dtype)
          if want_xt else None)
    return xr, xt


def _ptr(t: Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


@dataclass(frozen=True)
class HipOrthogonalize:
    """One Newton-Schulz kind on the HIP kernels.

    The optimizer feeds it straight from the momentum pass (the fused path);
    called as a function it is the reference's ``Orthogonalize``.

    Attributes:
        kind: The ``NewtonSchulz`` kind.
        lib_kind: The library's kind code.
        dtype: Iteration dtype (float16 for Gram, bfloat16 for the quintics).
        norm_safety: The Frobenius norm is scaled by this before the input is divided by it.
    """

    kind: NewtonSchulz
    lib_kind: int
    dtype: torch.dtype
    norm_safety: float

    @property
    def elem(self) -> int:
        return _lib.elem_code(self.dtype)

    def __call__(self, matrix: Tensor, epsilon: float) -> Tensor:
        """Orthogonalize a ``[N, rows, cols]`` (or 2-D) batch; returns bfloat16.

        Raises:
            ValueError: For a tensor that is not 2-D or 3-D or not on a GPU.
        """
        if matrix.ndim not in (2, 3):
            raise ValueError(f"expected a 2-D or 3-D batch, got {tuple(matrix.shape)}")
        if not matrix.is_cuda:
            raise ValueError("the HIP orthogonalization needs a GPU tensor")
        batch3 = matrix if matrix.ndim == 3 else matrix.unsqueeze(0)
        blocks, rows, cols = (int(d) for d in batch3.shape)
        out = torch.empty(blocks, rows, cols, device=matrix.device, dtype=torch.bfloat16)
        if blocks == 0:
            return out if matrix.ndim == 3 else out[0]
        # float32, float16 and bfloat16 inputs are read as they are (their
        # conversion to float32 is exact); others are converted first.
        source = batch3 if batch3.dtype in _INPUT_ELEMS else batch3.to(torch.float32)
        source = source.contiguous()
        device = source.device
        stream = _lib.stream_handle(device)
        rowsq = _workspace.buffer(device, "ortho_rowsq", (blocks * rows,), torch.float32)
        den = _workspace.buffer(device, "ortho_den", (blocks,), torch.float32)
        xr, xt = prepared_inputs(self, device, blocks, rows, cols, "ortho_xr", "ortho_xt")
        _lib.call("dionw_normalize_input", source.data_ptr(), _INPUT_ELEMS[source.dtype], blocks,
                  rows, cols, self.norm_safety, float(epsilon), rowsq.data_ptr(), den.data_ptr(),
                  *padded_sides(rows, cols), self.elem, _ptr(xr), _ptr(xt), stream)
        run_newton_schulz(self, blocks, rows, cols, xr, xt, out, stream)
        return out if matrix.ndim == 3 else out[0]


@dataclass(frozen=True)
class NewtonSchulzCall:
    """The library arguments of one Newton-Schulz call (see ``newton_schulz_call``)."""

    kind: int
    blocks: int
    r: int
    c: int
    x: int
    xt: int
    r_real: int
    c_real: int
    out: int
    tall: int
    out_ld: int
    out_stride: int
    workspace: int
    workspace_bytes: int


def newton_schulz_call(
    ortho: HipOrthogonalize,
    blocks: int,
    rows: int,
    cols: int,
    xr: Tensor | None,
    xt: Tensor | None,
    out: Tensor,
    workspace_name: str = "ns_workspace",
) -> NewtonSchulzCall:
    """The arguments that iterate on prepared inputs and write ``out`` ([blocks, rows, cols] bf16).

    ``xr`` is the normalized input in the weight's orientation ([blocks,
    round8(rows), round8(cols)]) and ``xt`` its transpose; a tall block
    (rows > cols) iterates on the transpose. Either may be None where
    ``prepared_orientations`` says the iteration does not read it; the others
    are overwritten. The iteration's workspace is the named scratch buffer
    ``workspace_name``. The result holds device addresses only: ``xr``, ``xt``
    and ``out`` must stay alive until the call has been issued.

    Raises:
        ValueError: If an input the iteration reads is None.
    """
    tall = rows > cols
    p_pad, j_pad = padded_sides(rows, cols)
    if tall:
        x, x_t, r, c, r_real, c_real = xt, xr, j_pad, p_pad, cols, rows
    else:
        x, x_t, r, c, r_real, c_real = xr, xt, p_pad, j_pad, rows, cols
    if x is None or (x_t is None and r % 32 != 0):
        raise ValueError(f"newton_schulz_call: [{rows}, {cols}] blocks need the prepared "
                         f"inputs {prepared_orientations(rows, cols)} (weight orientation, "
                         "transpose)")
    lib = _lib.library()
    need = int(lib.dionw_newton_schulz_workspace(ortho.lib_kind, blocks, r, c))
    ws = _workspace.buffer(out.device, workspace_name, (need,), torch.uint8)
    return NewtonSchulzCall(ortho.lib_kind, blocks, r, c, x.data_ptr(),
                            0 if x_t is None else x_t.data_ptr(), r_real, c_real,
                            out.data_ptr(), int(tall), cols, rows * cols, ws.data_ptr(), need)


def run_newton_schulz(
    ortho: HipOrthogonalize,
    blocks: int,
    rows: int,
    cols: int,
    xr: Tensor | None,
    xt: Tensor | None,
    out: Tensor,
    stream: int,
) -> None:
    """Run the iteration on prepared inputs and write ``out`` (``newton_schulz_call``)."""
    run_newton_schulz_call(newton_schulz_call(ortho, blocks, rows, cols, xr, xt, out), stream)


def run_newton_schulz_call(a: NewtonSchulzCall, stream: int) -> None:
    """Issue one prepared call (``dionw_newton_schulz``)."""
    _lib.call("dionw_newton_schulz", a.kind, a.blocks, a.r, a.c, a.x, a.xt, a.r_real, a.c_real,
              a.out, a.tall, a.out_ld, a.out_stride, a.workspace, a.workspace_bytes, stream)


def group_launches(calls: list[NewtonSchulzCall]) -> int:
    """Product launches one grouped call over ``calls`` issues (from their shapes;
    ``dionw_newton_schulz_group_launches``)."""
    n = len(calls)

    def arr(ctype, field):
        return (ctype * max(n, 1))(*[getattr(c, field) for c in calls])

    launches = int(_lib.library().dionw_newton_schulz_group_launches(
        n, arr(ctypes.c_int32, "kind"), arr(ctypes.c_int64, "blocks"), arr(ctypes.c_int64, "r"),
        arr(ctypes.c_int64, "c"), arr(ctypes.c_int64, "r_real"), arr(ctypes.c_int64, "c_real")))
    if launches < 0:
        raise ValueError("dionw_newton_schulz_group_launches: invalid run shapes")
    return launches


def run_newton_schulz_group(calls: list[NewtonSchulzCall], stream: int) -> None:
    """Independent Newton-Schulz calls in grouped launches (``dionw_newton_schulz_group``);
    their workspaces must be distinct buffers."""
    if not calls:
        return
    n = len(calls)

    def arr(ctype, field):
        return (ctype * n)(*[getattr(c, field) for c in calls])

    _lib.call("dionw_newton_schulz_group", n, arr(ctypes.c_int32, "kind"),
              arr(ctypes.c_int64, "blocks"), arr(ctypes.c_int64, "r"), arr(ctypes.c_int64, "c"),
              arr(ctypes.c_void_p, "x"), arr(ctypes.c_void_p, "xt"),
              arr(ctypes.c_int64, "r_real"), arr(ctypes.c_int64, "c_real"),
              arr(ctypes.c_void_p, "out"), arr(ctypes.c_int32, "tall"),
              arr(ctypes.c_int64, "out_ld"), arr(ctypes.c_int64, "out_stride"),
              arr(ctypes.c_void_p, "workspace"), arr(ctypes.c_size_t, "workspace_bytes"),
              stream)


_KINDS: dict[NewtonSchulz, HipOrthogonalize] = {
    NewtonSchulz.GRAM: HipOrthogonalize(NewtonSchulz.GRAM, _GRAM, torch.float16, 1.0),
    NewtonSchulz.POLAR_EXPRESS: HipOrthogonalize(
        NewtonSchulz.POLAR_EXPRESS, _PE_CUBLAS, torch.bfloat16, 1.02
    ),
    NewtonSchulz.POLAR_EXPRESS_TRITON: HipOrthogonalize(
        NewtonSchulz.POLAR_EXPRESS_TRITON, _PE_TRITON, torch.bfloat16, 1.02
    ),
    NewtonSchulz.KELLER: HipOrthogonalize(NewtonSchulz.KELLER, _KELLER_CUBLAS, torch.bfloat16, 1.0),
    NewtonSchulz.KELLER_TRITON: HipOrthogonalize(
        NewtonSchulz.KELLER_TRITON, _KELLER_TRITON, torch.bfloat16, 1.0
    ),
}


def newton_schulz_fn(kind: NewtonSchulz) -> Orthogonalize:
    """The orthogonalization of ``kind``.

    Raises:
        RuntimeError: For an unhandled kind.
    """
    try:
        return _KINDS[NewtonSchulz(kind)]
    except KeyError:
        raise RuntimeError(f"Unhandled NewtonSchulz: {kind}") from None
