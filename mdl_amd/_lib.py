"""ctypes binding of libmdl_hip.so, the C ABI declared in include/mdl_hip.h.

The shared library is built in-tree (``mdl_amd/libmdl_hip.so``) by
``mdl_amd/build.py``.  Importing this module never builds anything; when the
library is missing every call raises ``RuntimeError`` -- there is no other
implementation of these operations in the package.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "libmdl_hip.so"

MDL_OK = 0
MDL_F32 = 0
MDL_BF16 = 1
MDL_POOL_NONE = 0
MDL_POOL_SUM = 1
MDL_POOL_MEAN = 2
MDL_FLAG_EXCLUDE_NULL = 1
MDL_FLAG_ROWS_BY_POSITION = 2
MDL_FLAG_IDS_FROM_OFFSETS = 4
MDL_CLASSES_UNSUPPORTED = 0x80000000
ABI_VERSION = 6
MDL_BUCKET_PRE_HASHED = 0
MDL_BUCKET_MOD = 1
MDL_BUCKET_NONE = 2
MDL_TRUNCATE_HEAD = 0
MDL_TRUNCATE_TAIL = 1
MDL_SEQ_OLDEST_TO_NEWEST = 0
MDL_SEQ_NEWEST_TO_OLDEST = 1

# Host images of the C structs (field order and sizes match the header).
FEATURE_DTYPE = np.dtype(
    [
        ("weight", "<u8"),
        ("state", "<u8"),
        ("out", "<u8"),
        ("grad", "<u8"),
        ("num_rows", "<i8"),
        ("out_stride", "<i8"),
        ("row_base", "<i8"),
        ("payload_base", "<i8"),
        ("ids_begin", "<i8"),
        ("num_ids", "<i8"),
        ("bag_base", "<i8"),
        ("num_bags", "<i8"),
        ("dim", "<i4"),
        ("wdtype", "<i4"),
        ("odtype", "<i4"),
        ("pooling", "<i4"),
        ("flags", "<i4"),
        ("padding_idx", "<i4"),
        ("table", "<i4"),
        ("reserved", "<i4"),
    ]
)
CHUNK_DTYPE = np.dtype([("feature", "<i4"), ("count", "<i4"), ("first", "<i8")])
SPAN_DTYPE = np.dtype([("data", "<u8"), ("numel", "<i8"), ("dtype", "<i4"), ("row_elems", "<i4"),
                       ("live_rows", "<u8")])
TABLE_DTYPE = np.dtype(
    [
        ("weight", "<u8"),
        ("state", "<u8"),
        ("num_rows", "<i8"),
        ("row_base", "<i8"),
        ("dim", "<i4"),
        ("wdtype", "<i4"),
        ("feature", "<i4"),
        ("gdtype", "<i4"),
    ]
)
UPDATE_DTYPE = np.dtype(
    [
        ("weight", "<u8"),
        ("state", "<u8"),
        ("rows", "<u8"),
        ("values", "<u8"),
        ("count", "<u8"),
        ("num_rows", "<i8"),
        ("capacity", "<i8"),
        ("weight_stride", "<i8"),
        ("values_stride", "<i8"),
        ("unit_first", "<i8"),
        ("dim", "<i4"),
        ("wdtype", "<i4"),
        ("vdtype", "<i4"),
        ("lr", "<f4"),
    ]
)
MDL_UPDATE_UNIT = 256
assert UPDATE_DTYPE.itemsize == 96
assert FEATURE_DTYPE.itemsize == 128
assert CHUNK_DTYPE.itemsize == 16
assert SPAN_DTYPE.itemsize == 32
assert TABLE_DTYPE.itemsize == 48

_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_U32 = ctypes.c_uint32
_SZ = ctypes.c_size_t
_F = ctypes.c_float

# name -> (restype, argtypes)
SIGNATURES: dict[str, tuple] = {
    "mdl_last_error": (ctypes.c_char_p, []),
    "mdl_abi_version": (_I32, []),
    "mdl_bucketize": (_I32, [_P, _P, _I64, _I64, _I32, _I32, _P, _P, _P]),
    "mdl_bag_truncate_workspace_bytes": (_SZ, [_I64]),
    "mdl_bag_truncate": (
        _I32,
        [_P, _P, _I64, _P, _P, _I64, _I64, _I32, _I32, _I64, _I32, _P, _P, _P, _I64, _P, _P, _SZ, _P],
    ),
    "mdl_offsets_workspace_bytes": (_SZ, [_I64]),
    "mdl_lengths_to_offsets": (_I32, [_P, _I64, _P, _P, _SZ, _P]),
    "mdl_plan_chunks": (_I64, [_P, _I32, _I32, _P, _I64]),
    "mdl_forward": (_I32, [_P, _I32, _P, _I64, _P, _I64, _P, _P, _P, _P, _U32, _P, _P, _U32, _P]),
    "mdl_pool_backward": (_I32, [_P, _I32, _P, _I64, _P, _I64, _P, _P, _U32, _P]),
    "mdl_feature_classes": (_U32, [_P, _I32]),
    "mdl_table_classes": (_U32, [_P, _I32]),
    "mdl_sequence_forward": (
        _I32,
        [_P, _P, _P, _I64, _I64, _I64, _I32, _P, _P, _P, _P, _P, _U32, _P, _P],
    ),
    "mdl_sort_workspace_bytes": (_SZ, [_I64]),
    "mdl_sort_pairs": (_I32, [_P, _P, _P, _P, _I64, _I32, _P, _SZ, _P, _P]),
    "mdl_unique_workspace_bytes": (_SZ, [_I64]),
    "mdl_unique": (_I32, [_P, _I64, _I32, _P, _P, _P, _P, _P, _SZ, _P]),
    "mdl_sparse_keys": (_I32, [_P, _I64, _I64, _I64, _I64, _I64, _P, _P, _U32, _P, _P]),
    "mdl_backward_workspace_bytes": (_SZ, [_I64, _I32, _I32]),
    "mdl_backward_adagrad": (
        _I32,
        [_P, _I32, _P, _I32, _I32, _P, _P, _I64, _P, _I32, _P, _F, _F, _P, _P, _SZ, _U32, _P],
    ),
    "mdl_backward_sort": (_I32, [_P, _I32, _I32, _P, _P, _I64, _P, _I32, _P, _SZ, _P]),
    "mdl_backward_apply": (
        _I32,
        [_P, _I32, _P, _I32, _I32, _P, _P, _I64, _I32, _P, _F, _F, _P, _P, _SZ, _U32, _P],
    ),
    "mdl_backward_sumsq": (
        _I32,
        [_P, _I32, _P, _I32, _I32, _P, _P, _I64, _I32, _P, _P, _P, _SZ, _U32, _P],
    ),
    "mdl_sumsq_workspace_bytes": (_SZ, [_I32]),
    "mdl_sumsq": (_I32, [_P, _I32, _P, _P, _SZ, _P]),
    "mdl_clip_coef": (_I32, [_P, _I32, _F, _P, _P, _P]),
    "mdl_scale": (_I32, [_P, _I32, _P, _P]),
    "mdl_backward_count": (_I32, [_P, _I32, _I32, _P, _P, _I64, _P, _I32, _P, _P, _SZ, _P]),
    "mdl_backward_coalesce": (
        _I32,
        [_P, _I32, _P, _I32, _I32, _P, _P, _I64, _I32, _P, _P, _P, _P, _P, _SZ, _U32, _P],
    ),
    "mdl_noalloc_scratch_bytes": (_SZ, []),
    "mdl_backward_adagrad_noalloc": (
        _I32,
        [_P, _I32, _P, _I32, _I32, _P, _P, _I64, _P, _I32, _P, _F, _F, _P, _U32, _P],
    ),
    "mdl_backward_pad": (_I32, [_P, _I32, _P, _P, _P, _P, _P, _I64, _P]),
    "mdl_update_classes": (_U32, [_P, _I32]),
    "mdl_grouped_rowwise_adagrad": (_I32, [_P, _P, _I32, _F, _P, _P]),
    "mdl_rowwise_adagrad": (
        _I32,
        [_P, _I32, _I64, _I32, _I64, _P, _P, _I64, _P, _I32, _I64, _F, _F, _P, _P],
    ),
}

_LIB: ctypes.CDLL | None = None


class MdlError(RuntimeError):
    """A libmdl_hip call returned an error code."""


def lib() -> ctypes.CDLL:
    """The loaded library; raises when it has not been built."""

    global _LIB
    if _LIB is not None:
        return _LIB
    path = os.environ.get("MDL_HIP_LIB", str(LIB_PATH))
    if not os.path.exists(path):
        raise RuntimeError(
            f"libmdl_hip.so not found at {path}; build it with "
            "`python mdl_amd/build.py` (hipcc, gfx950)"
        )
    handle = ctypes.CDLL(path)
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = restype
        fn.argtypes = argtypes
    found = int(handle.mdl_abi_version())
    if found != ABI_VERSION:
        raise RuntimeError(
            f"{path} implements C ABI version {found}, this package binds version {ABI_VERSION}; "
            "rebuild it with `python mdl_amd/build.py`"
        )
    _LIB = handle
    return handle


def check(rc: int, what: str) -> None:
    if rc != MDL_OK:
        message = lib().mdl_last_error()
        text = message.decode() if message else ""
        raise MdlError(f"{what} failed ({rc}): {text}")
