"""Loader for ``libqsrt_amd.so`` (the C-ABI HIP library).

The library is built in-tree by ``__graft_entry__.build()`` (``make -C
qsrt_amd/csrc``) into ``qsrt_amd/_build``.  There is no fallback: every
GPU entry point raises if the library is missing or a call fails.

``torch`` is imported first on purpose: its ROCm wheel ships its own
``libamdhip64.so`` with the same SONAME as ``/opt/rocm``'s, so loading the
library after torch binds it to the runtime torch already initialised and
device pointers / streams are shared.
"""

from __future__ import annotations

import ctypes
from functools import lru_cache
from pathlib import Path

import torch  # noqa: F401  (must be loaded before the HIP library)

LIB_PATH = Path(__file__).resolve().parent / "_build" / "libqsrt_amd.so"

_c_void_p = ctypes.c_void_p
_c_int = ctypes.c_int
_c_i64 = ctypes.c_int64
_c_size = ctypes.c_size_t

# name -> (restype, argtypes); the single source of truth for the Python side
# of include/qsrt_amd.h.
SIGNATURES: dict[str, tuple] = {
    "qsrt_abi_version": (_c_int, []),
    "qsrt_last_error": (ctypes.c_char_p, []),
    "qsrt_viterbi_workspace_bytes": (_c_size, [_c_int, _c_i64]),
    "qsrt_viterbi_tiles": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_i64, _c_int, _c_int, _c_void_p, _c_int, _c_void_p, _c_size, _c_void_p],
    ),
    "qsrt_viterbi_tiles_ex": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_i64, _c_int, _c_int, _c_void_p, _c_int, _c_int, _c_void_p, _c_size,
         _c_void_p],
    ),
    "qsrt_quantize_tiles_sqg": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_i64, _c_void_p, _c_size, _c_void_p, _c_size, _c_void_p, _c_int, _c_int,
         ctypes.c_double, _c_void_p],
    ),
    "qsrt_pack_edges": (_c_int, [_c_void_p, _c_i64, _c_int, _c_void_p, _c_void_p]),
    "qsrt_unpack_states": (_c_int, [_c_void_p, _c_i64, _c_int, _c_void_p, _c_void_p]),
    "qsrt_decode_workspace_bytes": (_c_size, [_c_int]),
    "qsrt_decode": (_c_int, [_c_void_p, _c_int, _c_int, _c_void_p, _c_int, _c_int, _c_void_p, _c_size, _c_void_p]),
    "qsrt_decode_prepare": (_c_int, [_c_void_p, _c_int, _c_int, _c_void_p, _c_size, _c_void_p, _c_void_p]),
    "qsrt_decode_execute": (_c_int, [_c_void_p, _c_void_p, _c_int, _c_int, _c_void_p]),
    "qsrt_decode_noalloc": (_c_int, [_c_void_p, _c_int, _c_int, _c_void_p, _c_int, _c_int, _c_void_p]),
    "qsrt_gemm_tn": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_float,
         _c_int, _c_void_p],
    ),
    "qsrt_gemm_tn_workspace_bytes": (
        _c_size,
        [_c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int],
    ),
    "qsrt_gemm_tn_ws": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_float,
         _c_int, _c_void_p, _c_size, _c_void_p],
    ),
    "qsrt_gemm_tn_f64": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
         ctypes.c_double, _c_void_p],
    ),
    "qsrt_gemm_tn_f64_batched": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
         _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_double, _c_void_p],
    ),
    "qsrt_chol_diag_block_f64": (
        _c_int, [_c_void_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_void_p, _c_void_p, _c_void_p],
    ),
    "qsrt_block_unit_lower_f64": (
        _c_int, [_c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_void_p],
    ),
    "qsrt_bakron_band_update_f32": (
        _c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                 _c_i64, _c_i64, _c_i64, _c_void_p],
    ),
    "qsrt_bakron_band_update_lower_f32": (
        _c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                 _c_i64, _c_i64, _c_i64, _c_void_p],
    ),
    "qsrt_ldlq_targets": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_i64,
         _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_void_p],
    ),
    "qsrt_ldlq_commit": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
         _c_void_p],
    ),
    "qsrt_hadamard": (
        _c_int,
        [_c_void_p, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p],
    ),
    "qsrt_hadamard_f64": (
        _c_int,
        [_c_void_p, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p],
    ),
}


class DecodeJob(ctypes.Structure):
    """``qsrt_decode_job`` of ``include/qsrt_amd.h``."""

    _fields_ = [
        ("words", _c_void_p),
        ("tile_row_stride", _c_i64),
        ("tile_col_stride", _c_i64),
        ("row_scale", _c_void_p),
        ("col_scale", _c_void_p),
        ("out", _c_void_p),
        ("out_ld", _c_i64),
        ("rows", _c_i64),
        ("cols", _c_i64),
        ("block_row_stride", _c_i64),
        ("block_col_stride", _c_i64),
    ]


class DecodePlanStruct(ctypes.Structure):
    """``qsrt_decode_plan`` of ``include/qsrt_amd.h``."""

    _fields_ = [
        ("jobs", _c_void_p),
        ("n_jobs", _c_int),
        ("K", _c_int),
        ("total_blocks", _c_i64),
    ]


class NativeError(RuntimeError):
    """A C-ABI entry point returned a non-zero status."""


@lru_cache(maxsize=1)
def lib() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"QSRT HIP library not found at {LIB_PATH}; build it with "
            "`python -c 'import __graft_entry__ as g; g.build()'` (make -C qsrt_amd/csrc)"
        )
    handle = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_GLOBAL)
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return handle


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().qsrt_last_error().decode(errors="replace")
        if rc == -1:
            raise ValueError(f"{what}: {msg}")
        raise NativeError(f"{what} failed ({rc}): {msg}")


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor) -> int:
    return t.data_ptr()
