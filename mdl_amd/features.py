"""Id bucketing and the CSR bag layout of categorical features.

Mirrors the reference's ``pre_hashed`` encoding (src/features.py:360-376,
vectorised in src/dataloader.py:8463-8493 and :10173-10186), its list
truncation (src/dataloader.py:8565-8665) and the benchmark's ``mod`` id rule
(src/benchmark.py:1246-1250).  Bucketing of id tensors runs on the GPU
(``mdl_bucketize``); the scalar function keeps the reference's Python API.
"""

from __future__ import annotations

from typing import Any, Sequence

import numpy as np
import torch
from torch import Tensor

from . import ops

INT64_MIN = -(1 << 63)
INT64_MAX = (1 << 63) - 1


def pre_hashed_bucket(value: Any, num_buckets: int) -> int:
    """Map one signed int64 hash by its unsigned low bits to ``[1, num_buckets]``."""

    if num_buckets <= 0 or num_buckets & (num_buckets - 1):
        raise ValueError("pre_hashed num_buckets must be a positive power of two")
    if isinstance(value, bool) or not isinstance(value, int):
        raise TypeError(f"pre_hashed value must be an int64, got {type(value).__name__}")
    if value < INT64_MIN or value > INT64_MAX:
        raise ValueError(f"pre_hashed value {value!r} is outside signed int64 range")
    if value == 0:
        raise ValueError("pre_hashed non-null value must not be zero")
    return (value & (num_buckets - 1)) + 1


def pre_hashed_bucket_tensor(
    raw: Tensor,
    num_buckets: int,
    *,
    valid: Tensor | None = None,
    validate_nonzero: bool = True,
    name: str = "feature",
) -> Tensor:
    """Bucket a device tensor of raw hashes; nulls (``valid == 0``) become 0.

    With ``validate_nonzero`` a non-null zero raises ``ValueError`` (one device
    sync, like the reference's pyarrow scan for zeros).
    """

    if num_buckets <= 0 or num_buckets & (num_buckets - 1):
        raise ValueError("pre_hashed num_buckets must be a positive power of two")
    err = torch.zeros(1, dtype=torch.int32, device=raw.device) if validate_nonzero else None
    out = ops.bucketize(
        raw, num_buckets, mode="pre_hashed", valid=valid, validate_nonzero=validate_nonzero, error_count=err
    )
    if err is not None and int(err.item()):
        raise ValueError(f"pre_hashed input {name!r} contains non-null zero values")
    return out


def mod_bucket_tensor(raw: Tensor, num_embeddings: int) -> Tensor:
    """``1 + ((raw - 1) mod (num_embeddings - 1))`` with Python floor-mod."""

    if num_embeddings <= 1:
        return torch.zeros_like(raw)
    return ops.bucketize(raw, num_embeddings, mode="mod", validate_nonzero=False)


def bag_csr(
    rows: Sequence[Sequence[int | None] | None],
    *,
    max_length: int | None = None,
    truncation: str = "tail",
) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Ragged lists -> flat raw values, their validity and per-row lengths.

    A null row has length 0; a null element stays in place as an invalid
    slot (bucketed to padding id 0).  ``head`` keeps the first ``max_length``
    elements of a row, ``tail`` the last (src/dataloader.py:8565-8604).
    """

    if truncation not in ("head", "tail"):
        raise ValueError(f"unsupported list truncation {truncation!r}")
    if max_length is not None and max_length < 0:
        raise ValueError(f"max_length must be non-negative, got {max_length}")
    flat: list[int] = []
    valid: list[int] = []
    lengths: list[int] = []
    for row in rows:
        items = [] if row is None else list(row)
        if max_length is not None and len(items) > max_length:
            items = items[:max_length] if truncation == "head" else items[len(items) - max_length:]
        lengths.append(len(items))
        for item in items:
            flat.append(0 if item is None else int(item))
            valid.append(0 if item is None else 1)
    return (
        np.asarray(flat, dtype=np.int64),
        np.asarray(valid, dtype=np.uint8),
        np.asarray(lengths, dtype=np.int64),
    )
