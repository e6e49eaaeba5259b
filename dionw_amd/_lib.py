"""Loader of ``libdionw_hip.so``, the C-ABI library of the HIP kernels.

The library is built in-tree (``python -m dionw_amd.csrc.build``). There is no
fallback: if it is missing, every entry point raises, so a GPU step never runs
anything but the HIP kernels. torch is imported first so that the library
binds to the HIP runtime torch has loaded.
"""

from __future__ import annotations

import ctypes
import threading
from collections.abc import Sequence
from pathlib import Path
from typing import Any

import torch

__all__ = [
    "F16",
    "BF16",
    "F32",
    "LibraryMissingError",
    "call",
    "elem_code",
    "library",
    "library_path",
    "ptr",
    "ptr_array",
    "stream_handle",
]

F16, BF16, F32 = 0, 1, 2

_PATH = Path(__file__).resolve().parent / "libdionw_hip.so"
_LOCK = threading.Lock()
_LIB: ctypes.CDLL | None = None

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_f64 = ctypes.c_double
_pp = ctypes.POINTER(ctypes.c_void_p)
_pi64 = ctypes.POINTER(ctypes.c_int64)
_pi32 = ctypes.POINTER(ctypes.c_int32)
_psize = ctypes.POINTER(ctypes.c_size_t)

# name -> (restype, argtypes); mirrors include/dionw_hip.h.
SIGNATURES: dict[str, tuple[Any, list[Any]]] = {
    "dionw_last_error": (ctypes.c_char_p, []),
    "dionw_abi_version": (ctypes.c_int, []),
    "dionw_accumulate_scores": (ctypes.c_int, [_pp, _i32, _i64, _i64, _p, _p, _p, _i32, _p]),
    "dionw_full_sumsq": (ctypes.c_int, [_pp, _i32, _i64, _i64, _p, _f32, _i32, _p, _i32, _p]),
    "dionw_block_denom": (ctypes.c_int, [_p, _i64, _i64, _f32, _f32, _p, _i32, _p]),
    "dionw_normalize_input": (
        ctypes.c_int,
        [_p, _i32, _i64, _i64, _i64, _f32, _f32, _p, _p, _i64, _i64, _i32, _p, _p, _p],
    ),
    "dionw_select_rows": (
        ctypes.c_int,
        [_p, _p, _i64, _i64, _i64, _f32, _f32, _p, _p, _p, _i32, _p],
    ),
    "dionw_prepare_ns_input": (
        ctypes.c_int,
        [_pp, _i32, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _i32, _i32, _i32,
         _p, _p, _p],
    ),
    "dionw_gemm_nt": (
        ctypes.c_int,
        [_i32, _i64, _i64, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _f32,
         _f32, _p, _i64, _i64, _p, _i64, _i64, _i32, _p],
    ),
    "dionw_newton_schulz_workspace": (ctypes.c_size_t, [_i32, _i64, _i64, _i64]),
    "dionw_ns_coefficients": (ctypes.c_int, [_i32, ctypes.POINTER(ctypes.c_double)]),
    "dionw_newton_schulz": (
        ctypes.c_int,
        [_i32, _i64, _i64, _i64, _p, _p, _i64, _i64, _p, _i32, _i64, _i64, _p,
         ctypes.c_size_t, _p],
    ),
    "dionw_newton_schulz_group": (
        ctypes.c_int,
        [_i32, _pi32, _pi64, _pi64, _pi64, _pp, _pp, _pi64, _pi64, _pp, _pi32, _pi64, _pi64,
         _pp, _psize, _p],
    ),
    "dionw_newton_schulz_group_launches": (
        ctypes.c_int64, [_i32, _pi32, _pi64, _pi64, _pi64, _pi64, _pi64],
    ),
    "dionw_normuon_stats": (
        ctypes.c_int,
        [_p, _i64, _i64, _i64, _i64, _p, _p, _f32, _f32, _p, _p, _p, _p],
    ),
    "dionw_normuon_stats_noalloc": (
        ctypes.c_int,
        [_p, _i64, _i64, _i64, _i64, _p, _p, _f32, _f32, _p, _p, _p],
    ),
    "dionw_apply_update": (
        ctypes.c_int,
        [_pp, _i32, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _p, _f32, _f32, _i32, _p],
    ),
    "dionw_apply_update_ema": (
        ctypes.c_int,
        [_pp, _pp, _i32, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _p, _f32, _f32, _i32, _f32, _p],
    ),
    "dionw_apply_update_stage": (
        ctypes.c_int,
        [_pp, _pp, _i32, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _p, _f32, _f32, _i32, _p],
    ),
    "dionw_increment_steps": (ctypes.c_int, [_pp, _i32, _p]),
    "dionw_adamw": (
        ctypes.c_int,
        [_pp, _pp, _pp, _pp, _pp, _pi64, _i32, _f64, _f64, _f64, _f64, _f64, _p],
    ),
    "dionw_adamw_ema": (
        ctypes.c_int,
        [_pp, _pp, _pp, _pp, _pp, _pp, _pi64, _i32, _f64, _f64, _f64, _f64, _f64, _f32, _p],
    ),
    "dionw_ema_update": (ctypes.c_int, [_pp, _pp, _pi64, _i32, _f32, _i32, _p]),
}


class LibraryMissingError(RuntimeError):
    """The HIP library is not built (or cannot be loaded)."""


def library_path() -> Path:
    """Path of the in-tree shared library."""
    return _PATH


def library() -> ctypes.CDLL:
    """Load the library once and declare every entry point.

    Raises:
        LibraryMissingError: If the library is absent or fails to load.
    """
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is None:
            if not _PATH.exists():
                raise LibraryMissingError(
                    f"{_PATH} is not built: run `python -m dionw_amd.csrc.build` "
                    "(dionw_amd has no non-HIP fallback)"
                )
            try:
                lib = ctypes.CDLL(str(_PATH))
            except OSError as exc:
                raise LibraryMissingError(f"cannot load {_PATH}: {exc}") from exc
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _LIB = lib
    return _LIB


def call(name: str, *args: Any) -> None:
    """Call an entry point and turn a nonzero return code into an exception.

    Raises:
        ValueError: For a rejected argument (code 1).
        RuntimeError: For a failed launch (code 2).
    """
    lib = library()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        message = lib.dionw_last_error().decode(errors="replace")
        if rc == 1:
            raise ValueError(f"{name}: {message}")
        raise RuntimeError(f"{name}: {message}")


def ptr(tensor: torch.Tensor | None) -> int | None:
    """Device address of a tensor (None for None)."""
    return None if tensor is None else tensor.data_ptr()


def ptr_array(tensors: Sequence[torch.Tensor]) -> ctypes.Array[ctypes.c_void_p]:
    """A host array of the tensors' device addresses."""
    return (ctypes.c_void_p * max(len(tensors), 1))(*[t.data_ptr() for t in tensors])


def int64_array(values: Sequence[int]) -> ctypes.Array[ctypes.c_int64]:
    """A host array of int64 values."""
    return (ctypes.c_int64 * max(len(values), 1))(*values)


def stream_handle(device: torch.device | None = None) -> int:
    """The raw HIP stream of torch's current stream on ``device``."""
    return torch.cuda.current_stream(device).cuda_stream


def elem_code(dtype: torch.dtype) -> int:
    """The library's element code of a 16-bit or float32 dtype.

    Raises:
        ValueError: For other dtypes.
    """
    if dtype == torch.float16:
        return F16
    if dtype == torch.bfloat16:
        return BF16
    if dtype == torch.float32:
        return F32
    raise ValueError(f"unsupported dtype {dtype}")
