"""Id bucketing and the CSR bag layout of categorical features.

Mirrors the reference's ``pre_hashed`` encoding (src/features.py:360-376,
vectorised in src/dataloader.py:8463-8493 and :10173-10186), its list
truncation (src/dataloader.py:8565-8665) and the benchmark's ``mod`` id rule
(src/benchmark.py:1246-1250).  Bucketing of id tensors runs on the GPU
(``mdl_bucketize``; host tensors take the op's CPU kernel), and so does a
list feature's whole truncation, flatten and bucketing (``mdl_bag_truncate``:
:func:`bag_csr_tensor`, :func:`bag_csr_arrow`); the scalar function keeps the
reference's Python API.
"""

from __future__ import annotations

from typing import Any, Sequence

import numpy as np
import torch
from torch import Tensor

from . import library, ops  # noqa: F401  (library: the mdl_hip ops)

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
    """Bucket a tensor of raw int64 hashes; nulls (``valid == 0``) become 0.

    Runs the ``mdl_hip::bucketize`` op: the HIP kernel for a ROCm tensor, the
    op's CPU kernel for a host tensor (the reference buckets on the host,
    src/dataloader.py:8463-8493).  With ``validate_nonzero`` a non-null zero
    raises ``ValueError`` (one read of the zero count, like the reference's
    pyarrow scan for zeros).
    """

    if num_buckets <= 0 or num_buckets & (num_buckets - 1):
        raise ValueError("pre_hashed num_buckets must be a positive power of two")
    out, err = torch.ops.mdl_hip.bucketize(raw, valid, int(num_buckets), "pre_hashed", bool(validate_nonzero))
    if validate_nonzero and int(err.item()):
        raise ValueError(f"pre_hashed input {name!r} contains non-null zero values")
    return out


def mod_bucket_tensor(raw: Tensor, num_embeddings: int) -> Tensor:
    """``1 + ((raw - 1) mod (num_embeddings - 1))`` with Python floor-mod, and
    zeros for a table of one row (src/benchmark.py:1232-1233,1246-1250); on
    either device, through the ``mdl_hip::bucketize`` op."""

    if num_embeddings <= 1:
        return torch.zeros_like(raw)
    return torch.ops.mdl_hip.bucketize(raw, None, int(num_embeddings), "mod", False)[0]


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


def bag_csr_tensor(
    values: Tensor,
    offsets: Tensor,
    *,
    valid: Tensor | None = None,
    row_valid: Tensor | None = None,
    max_length: int | None = None,
    truncation: str = "tail",
    bucket: str = "none",
    num_buckets: int = 0,
    validate_nonzero: bool = True,
    name: str = "feature",
    exact: bool = True,
) -> dict[str, Tensor]:
    """A list feature in Arrow layout -> ``{"values", "lengths"}``, the CSR bag
    of ``_tensorize_categorical_bag`` (src/dataloader.py:8607-8665): rows
    truncated to ``max_length`` (``head``/``tail``, :8565-8604), nulls as
    length 0, flattened and bucketed (``bucket``: ``none`` for ids already
    encoded, ``pre_hashed`` or ``mod``) in one ``mdl_hip::bag_truncate`` call
    -- on the device for ROCm tensors, vectorised PyTorch on the CPU.

    ``exact`` (the reference's contract) sizes ``values`` to the kept total
    and raises the reference's errors, at the cost of one host read;
    ``exact=False`` returns the capacity-sized ids (zeros past the total),
    ``"offsets"`` whose last entry is the total, and ``"errors"`` (device
    int32) without reading anything back.
    """

    if truncation not in ops.TRUNCATIONS:
        raise ValueError(f"unsupported list truncation {truncation!r}")
    if max_length is not None and max_length < 0:
        raise ValueError(f"max_length must be non-negative, got {max_length}")
    if bucket == "pre_hashed" and (num_buckets <= 0 or num_buckets & (num_buckets - 1)):
        raise ValueError("pre_hashed num_buckets must be a positive power of two")
    ids, lengths, out_offsets, err = torch.ops.mdl_hip.bag_truncate(
        values, offsets, valid, row_valid, -1 if max_length is None else int(max_length), truncation, bucket,
        int(num_buckets), bool(validate_nonzero))
    if not exact:
        return {"values": ids, "lengths": lengths, "offsets": out_offsets, "errors": err}
    total, bad = (int(x) for x in torch.stack([out_offsets[-1], err[0].to(torch.int64)]).cpu())
    if bad:
        n = values.numel()
        malformed = bool(((offsets < 0) | (offsets > n)).any()) or bool((offsets[1:] < offsets[:-1]).any())
        if malformed:
            raise ValueError(f"list feature {name!r} has offsets outside its values")
        raise ValueError(f"pre_hashed input {name!r} contains non-null zero values")
    return {"values": ids[:total], "lengths": lengths}


def bag_csr_arrow(array: Any, *, device: torch.device | str = "cpu", **kwargs: Any) -> dict[str, Tensor]:
    """:func:`bag_csr_tensor` of a pyarrow list array (``ListArray``,
    ``LargeListArray`` or a chunked one): its offsets, values and validity
    bitmaps are read as numpy and moved to ``device`` once."""

    import pyarrow as pa
    import pyarrow.compute as pc

    if isinstance(array, pa.ChunkedArray):
        array = array.combine_chunks()
    offsets = array.offsets.to_numpy(zero_copy_only=False).astype(np.int64, copy=False)
    child = array.values
    raw = pc.fill_null(child, 0).to_numpy(zero_copy_only=False).astype(np.int64, copy=False)
    valid = child.is_valid().to_numpy(zero_copy_only=False).astype(np.uint8) if child.null_count else None
    row_valid = array.is_valid().to_numpy(zero_copy_only=False).astype(np.uint8) if array.null_count else None
    to = lambda a: None if a is None else torch.from_numpy(np.array(a)).to(device)  # noqa: E731
    return bag_csr_tensor(to(raw), to(offsets), valid=to(valid), row_valid=to(row_valid), **kwargs)
