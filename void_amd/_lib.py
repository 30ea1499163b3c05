"""ctypes binding of ``libvoid_amd.so`` (declared in ``include/void_amd.h``).

The library is the only compute path of this package: when it is missing the
SpMM entry points raise immediately instead of falling back to anything else.
"""

from __future__ import annotations

import ctypes
import threading
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_int64, c_size_t, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libvoid_amd.so")
ABI_VERSION = 5

# Scratch limits of void_spmm_int8_noalloc (VOID_NOALLOC_*_BYTES)
NOALLOC_COUNTER_BYTES = 1 << 20
NOALLOC_PARTIAL_BYTES = 31 << 20

# enum void_epilogue
EPI_RAW_I32 = 0
EPI_ROW_MEAN = 1
EPI_PER_BLOCK = 2
EPILOGUES = {"raw_i32": EPI_RAW_I32, "row_mean": EPI_ROW_MEAN, "per_block": EPI_PER_BLOCK}

# enum void_dtype
DT_F32, DT_BF16, DT_F16, DT_I32 = 0, 1, 2, 3

# enum void_activation (codes of get_activation_code, void/fusion.py:77-91)
ACT_NONE, ACT_RELU, ACT_GELU, ACT_SILU = 0, 1, 2, 3

# enum void_status
STATUS_NAMES = {
    0: "VOID_OK",
    -1: "VOID_ERR_ARG",
    -2: "VOID_ERR_UNSUPPORTED",
    -3: "VOID_ERR_HIP",
    -4: "VOID_ERR_WORKSPACE",
    -5: "VOID_ERR_CAPACITY",
}


class BsrDesc(ctypes.Structure):
    _fields_ = [
        ("tiles", c_void_p),
        ("scales", c_void_p),
        ("row_ptr", c_void_p),
        ("col_idx", c_void_p),
        ("M", c_int32),
        ("K", c_int32),
        ("n_blocks", c_int32),
        ("n_block_rows", c_int32),
        ("per_tensor_a", c_int32),
        ("reserved", c_int32),
    ]


ITEM_INLINE_COLS = 24
ITEM_INTS = 8 + ITEM_INLINE_COLS


class WorkItem(ctypes.Structure):
    _fields_ = [(name, c_int32) for name in
                ("row", "begin", "end", "tile", "nchunks", "chunk", "slot", "reserved")] + [
                    ("cols", c_int32 * ITEM_INLINE_COLS)]


class Plan(ctypes.Structure):
    _fields_ = [
        ("items", c_void_p),
        ("n_items", c_int32),
        ("n_split_tiles", c_int32),
        ("n_slots", c_int32),
        ("chunk_tiles", c_int32),
    ]


class DenseArgs(ctypes.Structure):
    _fields_ = [
        ("b", c_void_p),
        ("ldb", c_int64),
        ("b_col_major", c_int32),
        ("N", c_int32),
        ("b_scale", c_float),
        ("b_scale_vec", c_void_p),
        ("bias", c_void_p),
        ("c", c_void_p),
        ("ldc", c_int64),
        ("out_dtype", c_int32),
        ("activation", c_int32),
        ("bias_per_row", c_int32),
        ("reserved", c_int32),
    ]


# Every symbol include/void_amd.h declares, with its ctypes signature.
SIGNATURES = {
    "void_abi_version": (c_int, []),
    "void_last_error": (c_char_p, []),
    "void_panel_width": (c_int, []),
    "void_device_info": (c_int, [POINTER(c_int32), POINTER(c_int32), POINTER(c_int32), POINTER(c_int32)]),
    "void_stream_capture_id": (c_int, [c_void_p, POINTER(ctypes.c_ulonglong)]),
    "void_streamk_plan": (c_int, [POINTER(c_int32), POINTER(c_int32), c_int32, c_int32,
                                  POINTER(WorkItem), c_int32, POINTER(c_int32), POINTER(c_int32),
                                  POINTER(c_int32)]),
    "void_workspace_bytes": (c_size_t, [c_int32, c_int32, c_int32]),
    "void_spmm_int8": (c_int, [POINTER(BsrDesc), POINTER(DenseArgs), c_int32, POINTER(Plan),
                               c_void_p, c_size_t, c_void_p]),
    "void_spmm_int8_noalloc": (c_int, [POINTER(BsrDesc), POINTER(DenseArgs), c_int32, POINTER(Plan), c_void_p]),
    "void_spmm_fp8": (c_int, [POINTER(BsrDesc), POINTER(DenseArgs), POINTER(Plan),
                              c_void_p, c_size_t, c_void_p]),
    "void_spmm_fp8_f32b": (c_int, [POINTER(BsrDesc), POINTER(DenseArgs), POINTER(Plan),
                                   c_void_p, c_size_t, c_void_p]),
    "void_spmm_fp8_b16": (c_int, [POINTER(BsrDesc), POINTER(DenseArgs), c_int32, POINTER(Plan),
                                  c_void_p, c_size_t, c_void_p]),
    "void_spmm_f32": (c_int, [POINTER(BsrDesc), POINTER(DenseArgs), POINTER(Plan),
                              c_void_p, c_size_t, c_void_p]),
    "void_spmm_bf16": (c_int, [POINTER(BsrDesc), POINTER(DenseArgs), POINTER(Plan),
                               c_void_p, c_size_t, c_void_p]),
    "void_spmm_f16": (c_int, [POINTER(BsrDesc), POINTER(DenseArgs), POINTER(Plan),
                              c_void_p, c_size_t, c_void_p]),
    "void_transpose_b8": (c_int, [c_void_p, c_int64, c_int32, c_int32, c_void_p, c_int64, c_void_p]),
    "void_quantize_b_i8": (c_int, [c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_void_p]),
    "void_quantize_tiles_i8": (c_int, [c_void_p, c_int32, c_void_p, c_void_p, c_void_p]),
    "void_quantize_tiles_fp8": (c_int, [c_void_p, c_int32, c_void_p, c_void_p, c_void_p, c_void_p]),
    "void_sddmm_f32": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_int32, c_int32,
                               c_int32, c_int32, c_void_p, c_int32, c_void_p]),
    "void_sddmm_rows_f32": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int32, c_void_p, c_void_p,
                                    c_int32, c_int32, c_int32, c_void_p, c_int32, c_void_p]),
    "void_sddmm_rows_bf16": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int32, c_void_p, c_void_p,
                                     c_int32, c_int32, c_int32, c_void_p, c_int32, c_void_p]),
    "void_sddmm_rows_f16": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int32, c_void_p, c_void_p,
                                    c_int32, c_int32, c_int32, c_void_p, c_int32, c_void_p]),
    "void_csr_workspace_bytes": (c_size_t, [c_int32, c_int32]),
    "void_csr_count_blocks": (c_int, [c_void_p, c_void_p, c_int32, c_int32, c_void_p, c_size_t, c_void_p,
                                      c_void_p]),
    "void_csr_to_tiles": (c_int, [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_void_p, c_size_t,
                                  ctypes.c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
}

_lock = threading.Lock()
_lib = None


class VoidLibraryError(RuntimeError):
    """A call into libvoid_amd.so returned an error status."""


def lib() -> ctypes.CDLL:
    """Load ``libvoid_amd.so`` once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build the gfx950 library first "
                    "(python -m void_amd.build). There is no fallback compute path.")
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            if handle.void_abi_version() != ABI_VERSION:
                raise RuntimeError(f"{LIB_PATH} has ABI {handle.void_abi_version()}, expected {ABI_VERSION}")
            _lib = handle
    return _lib


def check(status: int, what: str) -> None:
    if status != 0:
        msg = lib().void_last_error().decode(errors="replace")
        raise VoidLibraryError(f"{what} failed with {STATUS_NAMES.get(status, status)}: {msg}")


def panel_width() -> int:
    return int(lib().void_panel_width())
