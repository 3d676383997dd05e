"""Tensor-level entry points over the libmdl_hip C ABI.

PyTorch supplies device memory and the current HIP stream; every computation
below is a launch of a hand-written gfx950 kernel in ``libmdl_hip.so``.  All
launches go to ``torch.cuda.current_stream()`` and none of these functions
synchronises the device unless its docstring says so.
"""

from __future__ import annotations

import ctypes
import weakref
from dataclasses import dataclass, field
from typing import Sequence

import numpy as np
import torch
from torch import Tensor

from . import _lib
from ._lib import (
    CHUNK_DTYPE,
    FEATURE_DTYPE,
    MDL_BF16,
    MDL_F32,
    MDL_FLAG_EXCLUDE_NULL,
    MDL_FLAG_ROWS_BY_POSITION,
    MDL_POOL_MEAN,
    MDL_POOL_NONE,
    MDL_POOL_SUM,
    TABLE_DTYPE,
    check,
    lib,
)

POOLING_CODES = {"none": MDL_POOL_NONE, "sum": MDL_POOL_SUM, "mean": MDL_POOL_MEAN}
NULL_POLICIES = ("exclude", "include_as_padding")
# Ids per forward chunk at most: the forward stages up to 480 rows of a
# pooled chunk in LDS, and chunks of about that size balance each wave's
# fixed cost against the length of its walk.
FORWARD_TARGET_IDS = 480


def forward_target_ids(feats: np.ndarray) -> int:
    """Ids per forward chunk for this call: FORWARD_TARGET_IDS, or fewer (down
    to 96) when a small call would give fewer than ~3000 chunks -- a wave per
    chunk, and every CU needs several (c0, 0.4 M ids: 480 ids per chunk took
    the lookup 0.045 ms, 120 took 0.031 ms)."""

    n = int(np.asarray(feats["num_ids"], dtype=np.int64).sum()) if len(feats) else 0
    return max(96, min(FORWARD_TARGET_IDS, n // 3072))


def _require_device(t: Tensor, what: str) -> None:
    if t.device.type != "cuda":
        raise RuntimeError(
            f"{what} must live on a ROCm device; libmdl_hip has no host implementation"
        )


def _ptr(t: Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return MDL_F32
    if dtype == torch.bfloat16:
        return MDL_BF16
    raise TypeError(f"unsupported embedding dtype {dtype}; expected float32 or bfloat16")


def upload(host: np.ndarray, device: torch.device) -> Tensor:
    """Copy a host array to the device through pinned memory, without a sync."""

    raw = np.ascontiguousarray(host).view(np.uint8).reshape(-1)
    staged = torch.empty(raw.size, dtype=torch.uint8, pin_memory=True)
    staged.numpy()[:] = raw
    return staged.to(device, non_blocking=True)


def _workspace(nbytes: int, device: torch.device) -> Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def _aligned16(t: Tensor) -> bool:
    return t.data_ptr() % 16 == 0


def _row_major_aligned(t: Tensor) -> Tensor:
    """Contiguous rows whose start is 16-byte aligned (copies only if needed)."""

    if not t.is_contiguous():
        t = t.contiguous()
    if not _aligned16(t):
        t = t.clone()
    return t


# ------------------------------------------------------------- bucketing --


def bucketize(
    raw: Tensor,
    num_buckets: int,
    *,
    mode: str = "pre_hashed",
    valid: Tensor | None = None,
    validate_nonzero: bool = True,
    error_count: Tensor | None = None,
) -> Tensor:
    """Bucket raw int64 hashes on the device (src/features.py:360-376 rule).

    ``mode="pre_hashed"``: ``(uint64(raw) & (num_buckets-1)) + 1``, null -> 0.
    ``mode="mod"``: ``1 + floormod(raw - 1, num_buckets - 1)`` (the benchmark
    id rule of src/benchmark.py:1246-1250).  Non-null zeros are counted in
    ``error_count`` (a device int32 scalar) when ``validate_nonzero``.
    """

    _require_device(raw, "raw ids")
    if raw.dtype != torch.int64:
        raise TypeError("raw ids must be torch.int64")
    raw = raw.contiguous()
    out = torch.empty_like(raw)
    code = _lib.MDL_BUCKET_PRE_HASHED if mode == "pre_hashed" else _lib.MDL_BUCKET_MOD
    if mode not in ("pre_hashed", "mod"):
        raise ValueError("mode must be pre_hashed or mod")
    if valid is not None:
        valid = valid.to(device=raw.device, dtype=torch.uint8).contiguous()
    check(
        lib().mdl_bucketize(
            raw.data_ptr(),
            _ptr(valid),
            raw.numel(),
            int(num_buckets),
            code,
            1 if validate_nonzero else 0,
            out.data_ptr(),
            _ptr(error_count),
            _stream(raw.device),
        ),
        "mdl_bucketize",
    )
    return out


BUCKET_MODES = {"none": _lib.MDL_BUCKET_NONE, "pre_hashed": _lib.MDL_BUCKET_PRE_HASHED, "mod": _lib.MDL_BUCKET_MOD}
TRUNCATIONS = {"head": _lib.MDL_TRUNCATE_HEAD, "tail": _lib.MDL_TRUNCATE_TAIL}


def bag_truncate(
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
    error_count: Tensor | None = None,
) -> tuple[Tensor, Tensor, Tensor]:
    """List feature -> CSR bag on the device: ``(ids [n_in], lengths [rows],
    out_offsets [rows+1])``.

    Row r of the list array holds ``values[offsets[r]:offsets[r+1]]``
    (Arrow list layout); a null row (``row_valid == 0``) keeps nothing (under
    tail truncation it keeps the last elements of its offsets span, as the
    reference's rebuild from raw offsets does, src/dataloader.py:8583-8604), a null
    element (``valid == 0``) keeps its slot and becomes id 0.  ``max_length``
    keeps a row's first (``head``) or last (``tail``) elements
    (src/dataloader.py:8565-8604); the kept elements are bucketed
    (``bucket``: ``none``, ``pre_hashed`` or ``mod``, as :func:`bucketize`).
    ``ids`` is capacity-sized: the kept total is ``out_offsets[-1]`` (on the
    device) and entries past it are 0, so nothing is read back.
    """

    _require_device(values, "list values")
    if values.dtype != torch.int64 or offsets.dtype != torch.int64:
        raise TypeError("list values and offsets must be torch.int64")
    if bucket not in BUCKET_MODES:
        raise ValueError(f"bucket must be one of {sorted(BUCKET_MODES)}")
    if truncation not in TRUNCATIONS:
        raise ValueError(f"unsupported list truncation {truncation!r}")
    if max_length is not None and max_length < 0:
        raise ValueError(f"max_length must be non-negative, got {max_length}")
    device = values.device
    values = values.contiguous()
    offsets = offsets.to(device).contiguous()
    rows = int(offsets.numel()) - 1
    if rows < 0:
        raise ValueError("list offsets need at least one entry")
    if valid is not None:
        valid = valid.to(device=device, dtype=torch.uint8).contiguous()
    if row_valid is not None:
        row_valid = row_valid.to(device=device, dtype=torch.uint8).contiguous()
    n_in = int(values.numel())
    ids = torch.empty(n_in, dtype=torch.int64, device=device)
    lengths = torch.empty(max(rows, 0), dtype=torch.int64, device=device)
    out_offsets = torch.empty(rows + 1, dtype=torch.int64, device=device)
    ws = _workspace(lib().mdl_bag_truncate_workspace_bytes(rows), device)
    check(
        lib().mdl_bag_truncate(
            offsets.data_ptr(), _ptr(row_valid), rows, _ptr(values) if n_in else None, _ptr(valid), n_in,
            -1 if max_length is None else int(max_length), TRUNCATIONS[truncation], BUCKET_MODES[bucket],
            int(num_buckets), 1 if validate_nonzero else 0, _ptr(lengths) if rows else None,
            out_offsets.data_ptr(), _ptr(ids) if n_in else None, n_in, _ptr(error_count), ws.data_ptr(),
            ws.numel(), _stream(device),
        ),
        "mdl_bag_truncate",
    )
    return ids, lengths, out_offsets


def lengths_to_offsets(lengths: Tensor) -> Tensor:
    """``[0, cumsum(lengths)]`` as int64 on the device."""

    _require_device(lengths, "lengths")
    lengths = lengths.to(torch.int64).contiguous()
    n = lengths.numel()
    offsets = torch.empty(n + 1, dtype=torch.int64, device=lengths.device)
    ws = _workspace(lib().mdl_offsets_workspace_bytes(n), lengths.device)
    check(
        lib().mdl_lengths_to_offsets(
            lengths.data_ptr(), n, offsets.data_ptr(), ws.data_ptr(), ws.numel(), _stream(lengths.device)
        ),
        "mdl_lengths_to_offsets",
    )
    return offsets


# ---------------------------------------------------------------- unique --


def unique(ids: Tensor, key_bits: int | None = None) -> tuple[Tensor, Tensor, Tensor]:
    """``torch.unique(ids, sorted=True, return_inverse=True, return_counts=True)``.

    Ids must be non-negative and below ``2**key_bits`` (default: the bit
    length of ``ids.max()``, which costs one device sync).  Returns
    ``(unique, inverse, counts)``; syncs once to size ``unique``.
    """

    _require_device(ids, "ids")
    ids = ids.to(torch.int64).contiguous()
    n = ids.numel()
    device = ids.device
    if key_bits is None:
        key_bits = int(ids.max().item()).bit_length() if n else 0
    uniq = torch.empty(n, dtype=torch.int64, device=device)
    inverse = torch.empty(n, dtype=torch.int64, device=device)
    counts = torch.empty(n, dtype=torch.int64, device=device)
    num = torch.zeros(1, dtype=torch.int64, device=device)
    ws = _workspace(lib().mdl_unique_workspace_bytes(n), device)
    check(
        lib().mdl_unique(
            ids.data_ptr(), n, int(key_bits), uniq.data_ptr(), inverse.data_ptr(), counts.data_ptr(),
            num.data_ptr(), ws.data_ptr(), ws.numel(), _stream(device),
        ),
        "mdl_unique",
    )
    u = int(num.item())
    return uniq[:u], inverse.view(ids.shape), counts[:u]


# --------------------------------------------------------------- adagrad --


def rowwise_adagrad_(
    weight: Tensor,
    accumulator: Tensor,
    rows: Tensor,
    values: Tensor,
    *,
    lr: float,
    eps: float,
    error_count: Tensor | None = None,
) -> None:
    """In-place row-wise Adagrad on unique rows (src/optim.py:68-108)."""

    _require_device(weight, "weight")
    if weight.ndim != 2:
        raise ValueError("row-wise Adagrad expects a 2D weight")
    n = rows.numel()
    if n == 0:
        return
    if accumulator.dtype != torch.float32 or not accumulator.is_contiguous():
        raise TypeError("row-wise Adagrad accumulator must be a contiguous float32 tensor")
    if weight.stride(1) != 1:
        raise ValueError("weight rows must be contiguous")
    rows = rows.to(torch.int64).contiguous()
    if weight.dtype == torch.float32 and values.dtype != torch.float32:
        values = values.float()
    if values.dtype not in (torch.float32, torch.bfloat16):
        values = values.float()
    values = _row_major_aligned(values)
    check(
        lib().mdl_rowwise_adagrad(
            weight.data_ptr(), dtype_code(weight.dtype), weight.size(0), weight.size(1), weight.stride(0),
            accumulator.data_ptr(), rows.data_ptr(), n, values.data_ptr(), dtype_code(values.dtype),
            values.stride(0), float(lr), float(eps), _ptr(error_count), _stream(weight.device),
        ),
        "mdl_rowwise_adagrad",
    )


# ------------------------------------------------------------- grouping --


@dataclass
class TableSpec:
    weight: Tensor
    state: Tensor | None
    row_base: int


@dataclass
class FeatureSpec:
    """One lookup request of a grouped call."""

    table: int
    pooling: int
    exclude_null: bool
    padding_idx: int
    out_dtype: torch.dtype
    rows_by_position: bool = False


# Sort keys are 32-bit: the rows of one key group stay below this, and a key
# of the group's row count marks ids that receive no gradient.
KEY_SPACE = 0xFFFFFFFF


@dataclass
class KeyGroup:
    """Features ``[lo, hi)`` of a plan and the tables they read, whose rows
    share one 32-bit key space (one sort and one segment reduce).

    ``plan`` is the group as a plan of its own: the same table specs (their
    ``row_base`` counted within the group) and features, table indices
    renumbered in ``tables`` order.  A group that is the whole plan refers to
    it weakly, so a plan and its groups form no reference cycle that would
    keep its tables alive until the next garbage collection."""

    lo: int
    hi: int
    tables: list[int]
    rows: int
    _plan: object

    @property
    def plan(self) -> "GroupPlan":
        p = self._plan
        return p() if isinstance(p, weakref.ref) else p


class GroupPlan:
    """Tables and features of a grouped lookup; static across steps.

    Features that pass the same weight tensor share one table.  Sort keys of
    table t are ``row_base[t] + id``; the key ``sentinel`` (at least the rows of
    every key group) marks ids that receive no gradient.

    Keys are 32-bit.  A plan of 2^32 - 1 rows or more in all is cut into key
    groups (:attr:`groups`): runs of consecutive features whose tables hold
    fewer rows than that together, each table's rows counted from its group's
    first.  One forward still looks up every feature; each group then has a
    sort and a reduce of its own over its features' stretch of the keys.  A
    table's features must then follow one another closely enough that no other
    group's features come between them, and one table stays below 2^32 - 1
    rows.
    """

    def __init__(self) -> None:
        self.tables: list[TableSpec] = []
        self.features: list[FeatureSpec] = []
        self._table_of_ptr: dict[int, int] = {}
        self.total_rows = 0
        self._groups: list[KeyGroup] | None = None
        self._groups_for: tuple[int, int] = (-1, -1)
        # Host arrays derived from this layout alone (addresses, sizes and
        # codes, no tensor references), shared by every plan of the same
        # layout when the plan comes from ``memoized_plan``.
        self._memo: dict | None = None

    def add_table(self, weight: Tensor, state: Tensor | None = None, *, shared: bool = True) -> int:
        key = weight.data_ptr()
        if shared and key in self._table_of_ptr:
            t = self._table_of_ptr[key]
            if state is not None and self.tables[t].state is None:
                self.tables[t].state = state
            return t
        if weight.ndim != 2 or weight.stride(1) != 1 or weight.stride(0) != weight.size(1):
            raise ValueError("embedding weights must be contiguous [rows, dim] tensors")
        dtype_code(weight.dtype)
        _require_device(weight, "embedding weight")
        t = len(self.tables)
        self.tables.append(TableSpec(weight=weight, state=state, row_base=self.total_rows))
        if shared:
            self._table_of_ptr[key] = t
        if int(weight.size(0)) >= KEY_SPACE:
            raise ValueError("a table of a grouped lookup holds fewer than 2^32 - 1 rows")
        self.total_rows += int(weight.size(0))
        return t

    def add_feature(
        self,
        weight: Tensor,
        *,
        pooling: str = "none",
        null_policy: str = "exclude",
        padding_idx: int = 0,
        state: Tensor | None = None,
        out_dtype: torch.dtype | None = None,
        rows_by_position: bool = False,
    ) -> int:
        """Add one lookup request; ``rows_by_position`` pools the rows of an
        already-embedded ``weight`` (row i = id slot i) instead of looking up
        ids, which then only decide the null weights."""

        if pooling not in POOLING_CODES:
            raise ValueError(f"unsupported pooling {pooling!r}")
        if null_policy not in NULL_POLICIES:
            raise ValueError(f"unsupported categorical bag null policy {null_policy!r}")
        if rows_by_position and pooling == "none":
            raise ValueError("rows by position need a pooled feature")
        t = self.add_table(weight, state, shared=not rows_by_position)
        self.features.append(
            FeatureSpec(
                table=t,
                pooling=POOLING_CODES[pooling],
                exclude_null=null_policy == "exclude",
                padding_idx=int(padding_idx),
                out_dtype=out_dtype or weight.dtype,
                rows_by_position=bool(rows_by_position),
            )
        )
        return len(self.features) - 1

    @property
    def groups(self) -> list[KeyGroup]:
        """The key groups (one for a plan below 2^32 - 1 rows: every feature
        and table, row bases as added)."""

        shape = (len(self.tables), len(self.features))
        if self._groups is not None and self._groups_for == shape:
            return self._groups
        if self.total_rows < KEY_SPACE:
            groups = [KeyGroup(0, len(self.features), list(range(len(self.tables))), self.total_rows,
                               weakref.ref(self))]
            base = 0
            for t in self.tables:
                t.row_base = base
                base += int(t.weight.size(0))
        else:
            groups = self._split()
        self._groups, self._groups_for = groups, shape
        return groups

    def _split(self) -> list[KeyGroup]:
        cuts: list[tuple[int, int, list[int], int]] = []
        owner: dict[int, int] = {}
        lo, tabs, rows = 0, [], 0
        for f, spec in enumerate(self.features):
            t = spec.table
            if t in owner and owner[t] != len(cuts):
                raise ValueError(
                    "a plan of 2^32 - 1 rows or more needs each table's features in one run of features "
                    f"whose tables hold fewer rows than that (table {t} is read again by feature {f})"
                )
            if t in owner:
                continue
            r = int(self.tables[t].weight.size(0))
            if tabs and rows + r >= KEY_SPACE:
                cuts.append((lo, f, tabs, rows))
                lo, tabs, rows = f, [], 0
            owner[t] = len(cuts)
            tabs.append(t)
            rows += r
        cuts.append((lo, len(self.features), tabs, rows))
        groups = []
        for lo, hi, tabs, rows in cuts:
            sub = GroupPlan()
            local = {}
            base = 0
            for t in tabs:
                spec = self.tables[t]
                spec.row_base = base
                base += int(spec.weight.size(0))
                local[t] = len(sub.tables)
                sub.tables.append(spec)
            sub.total_rows = base
            for spec in self.features[lo:hi]:
                sub.features.append(FeatureSpec(
                    table=local[spec.table], pooling=spec.pooling, exclude_null=spec.exclude_null,
                    padding_idx=spec.padding_idx, out_dtype=spec.out_dtype, rows_by_position=spec.rows_by_position,
                ))
            groups.append(KeyGroup(lo, hi, tabs, rows, sub))
        return groups

    @property
    def split(self) -> bool:
        """Whether the plan needs more than one key group."""

        return len(self.groups) > 1

    @property
    def sentinel(self) -> int:
        return max(g.rows for g in self.groups) if self.groups else 0

    @property
    def key_bits(self) -> int:
        return max(1, int(self.sentinel).bit_length())

    @property
    def max_dim(self) -> int:
        return max(int(t.weight.size(1)) for t in self.tables)


@dataclass
class ForwardResult:
    """What a grouped forward leaves for its backward."""

    plan: GroupPlan
    device: torch.device
    ids: Tensor
    offsets: Tensor | None
    outputs: list[Tensor]
    feats: np.ndarray
    keys: Tensor | None
    payload: Tensor | None
    bag_count: Tensor | None
    error_count: Tensor
    keep: list = field(default_factory=list)
    count: int | None = None  # ids of the call when ``ids`` is not the concatenated array

    @property
    def num_ids(self) -> int:
        return int(self.ids.numel()) if self.count is None else int(self.count)


class _UploadCache:
    """Device copies of small host arrays, reused while their bytes repeat."""

    def __init__(self, capacity: int = 8) -> None:
        self.capacity = capacity
        self.entries: dict[bytes, Tensor] = {}

    def get(self, host: np.ndarray, device: torch.device) -> Tensor:
        key = host.tobytes()
        hit = self.entries.get(key)
        if hit is not None and hit.device == device:
            return hit
        dev = upload(host, device)
        if len(self.entries) >= self.capacity:
            self.entries.pop(next(iter(self.entries)))
        self.entries[key] = dev
        return dev


_CACHE = _UploadCache()


def _static_features(plan: GroupPlan) -> np.ndarray:
    """The descriptor columns that depend on the layout alone (tables,
    dims, dtypes, pooling, flags); the per-call columns are zero."""

    specs = plan.features
    nf = len(specs)
    tab = [plan.tables[s.table] for s in specs]
    feats = np.zeros(nf, dtype=FEATURE_DTYPE)
    feats["weight"] = [t.weight.data_ptr() for t in tab]
    feats["state"] = [t.state.data_ptr() if t.state is not None else 0 for t in tab]
    feats["num_rows"] = [int(t.weight.size(0)) for t in tab]
    feats["row_base"] = [t.row_base for t in tab]
    feats["dim"] = [int(t.weight.size(1)) for t in tab]
    feats["wdtype"] = [dtype_code(t.weight.dtype) for t in tab]
    feats["odtype"] = [dtype_code(s.out_dtype) for s in specs]
    feats["pooling"] = np.array([s.pooling for s in specs], dtype=np.int32)
    feats["flags"] = [
        (MDL_FLAG_EXCLUDE_NULL if s.exclude_null else 0) | (MDL_FLAG_ROWS_BY_POSITION if s.rows_by_position else 0)
        for s in specs
    ]
    feats["padding_idx"] = [s.padding_idx for s in specs]
    feats["table"] = [s.table for s in specs]
    for s, t in zip(specs, tab):
        if t.weight.dtype == torch.float32 and s.out_dtype != torch.float32:
            raise TypeError("float32 tables produce float32 outputs")
    return feats


def build_features(
    plan: GroupPlan,
    id_counts: Sequence[int],
    bag_counts: Sequence[int],
    out_ptrs: Sequence[int],
    out_strides: Sequence[int],
) -> np.ndarray:
    """Host image of the feature descriptors (vectorised over features).

    ``bag_counts[f]`` is the number of bags of a pooled feature (ignored for
    unpooled ones).  When any feature is pooled, every unpooled feature
    occupies one pseudo-bag in the offsets array (its whole id range), so the
    offsets of all features come from one scan over the concatenated lengths.
    """

    plan.groups  # row bases of a plan cut into key groups
    memo = plan._memo
    static = memo.get("feats") if memo is not None else None
    if static is None:
        static = _static_features(plan)
        if memo is not None:
            memo["feats"] = static
    nf = len(static)
    pooled = static["pooling"] != MDL_POOL_NONE
    pooled_any = bool(pooled.any())
    ids = np.asarray(id_counts, dtype=np.int64)
    bags = np.where(pooled, np.asarray(bag_counts, dtype=np.int64), 0)
    rows_out = np.where(pooled, bags, ids)
    bag_slots = np.where(pooled, bags, 1 if pooled_any else 0)
    feats = static.copy()
    feats["out"] = np.asarray(out_ptrs, dtype=np.uint64)
    feats["out_stride"] = np.asarray(out_strides, dtype=np.int64)
    if nf:
        feats["payload_base"][1:] = np.cumsum(rows_out)[:-1]
        feats["ids_begin"][1:] = np.cumsum(ids)[:-1]
        feats["bag_base"][1:] = np.cumsum(bag_slots)[:-1]
    feats["num_ids"] = ids
    feats["num_bags"] = bags
    if int(rows_out.sum()) >= 0xFFFFFFFF:
        raise ValueError("a grouped lookup supports fewer than 2^32 - 1 output rows")
    return feats


def forward_packed(
    plan: GroupPlan,
    all_ids: Tensor,
    offsets: Tensor | None,
    id_counts: Sequence[int],
    bag_counts: Sequence[int],
    outputs: Sequence[Tensor],
    *,
    with_backward: bool,
    error_count: Tensor | None = None,
    with_bag_count: bool | None = None,
) -> ForwardResult:
    """Grouped lookup over caller-packed buffers (no per-feature copies).

    ``all_ids``: every feature's ids back to back; ``offsets``: absolute bag
    bounds from one scan of the concatenated lengths (see build_features);
    ``outputs[f]``: row-major output rows of feature f (2-D views with unit
    column stride, e.g. column slices of one ``[B, sum(dim)]`` buffer).
    ``with_backward`` emits the backward's sort keys and bag counts;
    ``with_bag_count`` (default: ``with_backward``) only the bag counts.
    """

    device = all_ids.device
    stream = _stream(device)
    n = int(all_ids.numel())
    # Bags that are all empty still get zero rows: the kernel needs a real
    # address even when there are no ids (it reads none of them).
    ids_arg = all_ids if n else torch.zeros(1, dtype=torch.int64, device=device)
    out_ptrs = [o.data_ptr() for o in outputs]
    out_strides = [o.stride(0) if o.ndim == 2 else int(o.size(-1)) for o in outputs]
    feats = build_features(plan, id_counts, bag_counts, out_ptrs, out_strides)
    pooled_any = bool((feats["pooling"] != MDL_POOL_NONE).any())
    if pooled_any and offsets is None:
        raise ValueError("pooled features need offsets")
    target = forward_target_ids(feats)
    n_chunks = lib().mdl_plan_chunks(feats.ctypes.data, len(feats), target, None, 0)
    if n_chunks < 0:
        check(int(n_chunks), "mdl_plan_chunks")
    chunks = np.zeros(max(n_chunks, 1), dtype=CHUNK_DTYPE)
    lib().mdl_plan_chunks(feats.ctypes.data, len(feats), target, chunks.ctypes.data, n_chunks)
    feats_dev = _CACHE.get(feats, device)
    chunks_dev = _CACHE.get(chunks, device)
    if error_count is None:
        error_count = torch.zeros(1, dtype=torch.int32, device=device)
    keys = payload = bag_count = None
    total_rows_out = int(feats["payload_base"][-1] + (feats["num_bags"][-1] if feats["pooling"][-1] else feats["num_ids"][-1])) if len(feats) else 0
    if with_bag_count is None:
        with_bag_count = with_backward
    if with_backward:
        alloc = torch.empty if n else torch.zeros
        keys = alloc(max(n, 1), dtype=torch.int32, device=device)
        payload = alloc(max(n, 1), dtype=torch.int32, device=device)
    if with_bag_count and pooled_any:
        # zeros: the rows of unpooled features have no bag and are not written
        bag_count = torch.zeros(max(total_rows_out, 1), dtype=torch.float32, device=device)
    check(
        lib().mdl_forward(
            feats_dev.data_ptr(), len(feats), chunks_dev.data_ptr(), n_chunks, ids_arg.data_ptr(), n,
            _ptr(offsets), _ptr(keys), _ptr(payload), None, plan.sentinel, _ptr(bag_count),
            error_count.data_ptr(), feature_classes(feats), stream,
        ),
        "mdl_forward",
    )
    return ForwardResult(
        plan=plan, device=device, ids=all_ids, offsets=offsets, outputs=list(outputs), feats=feats,
        keys=keys, payload=payload, bag_count=bag_count, error_count=error_count,
        keep=[feats_dev, chunks_dev, ids_arg],
    )


def grouped_forward(
    plan: GroupPlan,
    ids: Sequence[Tensor],
    lengths: Sequence[Tensor | None],
    *,
    with_backward: bool,
    outputs: Sequence[Tensor] | None = None,
    error_count: Tensor | None = None,
    with_bag_count: bool | None = None,
) -> ForwardResult:
    """Look up (and pool) every feature of ``plan`` in one launch.

    ``ids[f]`` are feature f's ids (any shape for unpooled features, a flat
    CSR value list for pooled ones) and ``lengths[f]`` its bag lengths (None
    for unpooled features).  Outputs are ``[*ids.shape, dim]`` (unpooled) or
    ``[len(lengths), dim]`` (pooled) unless the caller passes ``outputs``.
    """

    specs = plan.features
    if len(ids) != len(specs) or len(lengths) != len(specs):
        raise ValueError("one ids tensor and one lengths entry per feature")
    device = plan.tables[0].weight.device
    id_counts = []
    bag_counts = []
    pooled_any = any(s.pooling != MDL_POOL_NONE for s in specs)
    for f, spec in enumerate(specs):
        t = ids[f]
        if t.dtype != torch.long:
            raise TypeError("sharded embedding indices must be torch.long")
        _require_device(t, "ids")
        id_counts.append(int(t.numel()))
        if spec.pooling != MDL_POOL_NONE:
            ln = lengths[f]
            if ln is None or ln.ndim != 1:
                raise ValueError("categorical bag lengths must have shape [B]")
            bag_counts.append(int(ln.numel()))
        else:
            bag_counts.append(0)
    length_parts = []
    if pooled_any:
        # the unpooled features' pseudo-lengths (their id counts) in one upload
        pseudo = [c for c, s in zip(id_counts, specs) if s.pooling == MDL_POOL_NONE]
        pseudo_dev = upload(np.asarray(pseudo, dtype=np.int64), device).view(torch.int64) if pseudo else None
        k = 0
        for f, spec in enumerate(specs):
            if spec.pooling != MDL_POOL_NONE:
                ln = lengths[f]
                length_parts.append(ln if ln.dtype == torch.int64 else ln.to(torch.int64))
            else:
                length_parts.append(pseudo_dev[k: k + 1])
                k += 1
    flat = [t.reshape(-1) for t in ids]
    all_ids = (flat[0] if len(flat) == 1 else torch.cat(flat)).contiguous()
    offsets = None
    if pooled_any:
        offsets = lengths_to_offsets(torch.cat(length_parts) if len(length_parts) > 1 else length_parts[0])
    if outputs is None:
        outputs = []
        for f, spec in enumerate(specs):
            dim = int(plan.tables[spec.table].weight.size(1))
            shape = (*ids[f].shape, dim) if spec.pooling == MDL_POOL_NONE else (bag_counts[f], dim)
            outputs.append(torch.empty(shape, dtype=spec.out_dtype, device=device))
    else:
        for f, spec in enumerate(specs):
            o = outputs[f]
            if o.stride(-1) != 1 or o.dtype != spec.out_dtype:
                raise ValueError("caller outputs must have unit column stride and the feature's dtype")
    return forward_packed(
        plan, all_ids, offsets, id_counts, bag_counts, outputs,
        with_backward=with_backward, error_count=error_count, with_bag_count=with_bag_count,
    )


def feature_classes(feats: np.ndarray) -> int:
    """Mask of the row-access classes present (which kernels to launch)."""

    return int(lib().mdl_feature_classes(feats.ctypes.data, len(feats)))


def table_classes(tables: np.ndarray) -> int:
    return int(lib().mdl_table_classes(tables.ctypes.data, len(tables)))


def lane_elems(dim: int, esize: int, vec: bool) -> int:
    """Elements one lane moves per row in the kernels (their width rule):
    one 16-byte vector of the weight type, doubled up to 8 elements while
    four lanes do not cover the row and the doubled width divides ``dim``;
    1 for rows that are not 16-byte aligned."""

    if not vec:
        return 1
    w = 1 if esize == 2 else 0
    while (8 << w) <= 8 and (4 << w) * 4 < dim and dim % (8 << w) == 0:
        w += 1
    return 4 << w


def _tables_array(plan: GroupPlan, feats: np.ndarray) -> np.ndarray:
    if plan.total_rows >= KEY_SPACE:
        raise ValueError("tables of 2^32 - 1 rows or more are keyed per key group (GroupPlan.groups)")
    memo = plan._memo
    key = ("tables", feats["odtype"].tobytes())
    if memo is not None and key in memo:
        return memo[key]
    tables = _build_tables_array(plan, feats)
    if memo is not None:
        tables.setflags(write=False)
        memo[key] = tables
    return tables


def _build_tables_array(plan: GroupPlan, feats: np.ndarray) -> np.ndarray:
    plan.groups  # row bases
    tables = np.zeros(len(plan.tables), dtype=TABLE_DTYPE)
    users: dict[int, list[int]] = {}
    for f, spec in enumerate(plan.features):
        users.setdefault(spec.table, []).append(f)
    for t, table in enumerate(plan.tables):
        w = table.weight
        rec = tables[t]
        rec["weight"] = w.data_ptr()
        rec["state"] = table.state.data_ptr() if table.state is not None else 0
        rec["num_rows"] = int(w.size(0))
        rec["row_base"] = table.row_base
        rec["dim"] = int(w.size(1))
        rec["wdtype"] = dtype_code(w.dtype)
        fs = users.get(t, [])
        rec["feature"] = fs[0] if len(fs) == 1 else -1
        gd = {int(feats[f]["odtype"]) for f in fs}
        if len(gd) > 1:
            raise TypeError("features that share a table must share an output dtype")
        rec["gdtype"] = gd.pop() if gd else dtype_code(w.dtype)
    return tables


def _attach_grads(res: ForwardResult, grads: Sequence[Tensor | None]) -> tuple[np.ndarray, list[Tensor]]:
    feats = res.feats.copy()
    keep = []
    gptr = []
    gstride = []
    for f, spec in enumerate(res.plan.features):
        out = res.outputs[f]
        g = grads[f]
        if g is None:
            g = torch.zeros_like(out)
        if g.dtype != spec.out_dtype:
            g = g.to(spec.out_dtype)
        dim = int(res.plan.tables[spec.table].weight.size(1))
        g2 = g if g.ndim == 2 else g.reshape(-1, dim)
        esize = g2.element_size()
        if (dim * esize) % 16 == 0 and (
            g2.stride(-1) != 1 or g2.data_ptr() % 16 != 0 or (g2.stride(0) * esize) % 16 != 0
        ):
            g2 = g2.contiguous()
            if g2.data_ptr() % 16 != 0:
                g2 = g2.clone()
        if g2.stride(-1) != 1:
            g2 = g2.contiguous()
        keep.append(g2)
        gptr.append(g2.data_ptr())
        gstride.append(g2.stride(0))
    feats["grad"] = np.asarray(gptr, dtype=np.uint64)
    feats["out_stride"] = np.asarray(gstride, dtype=np.int64)
    return feats, keep


def pool_backward(
    res: ForwardResult, grads: Sequence[Tensor | None], dests: Sequence[Tensor | None]
) -> None:
    """Per-position gradient of the pooled features of a forward (one launch).

    ``grads[f]`` is the upstream gradient of feature f's pooled output and
    ``dests[f]`` a contiguous ``[num_ids_f, dim]`` tensor of the weight dtype
    that receives ``grad[bag] * w_i / max(count, 1)`` (mean) or
    ``grad[bag] * w_i`` (sum) for every id position i; None skips feature f.
    The forward must have kept its bag counts.
    """

    if res.bag_count is None or res.offsets is None:
        raise RuntimeError("the forward ran without bag counts")
    feats = res.feats.copy()
    keep: list[Tensor] = []
    sel: list[int] = []
    for f, spec in enumerate(res.plan.features):
        d = dests[f]
        if d is None or spec.pooling == MDL_POOL_NONE:
            continue
        weight = res.plan.tables[spec.table].weight
        n_f = int(feats["num_ids"][f])
        dim = int(feats["dim"][f])
        if d.dtype != weight.dtype or not d.is_contiguous() or d.numel() != n_f * dim:
            raise ValueError("pool_backward destinations are contiguous [num_ids, dim] tensors of the weight dtype")
        g = grads[f]
        if g is None:
            g = torch.zeros_like(res.outputs[f])
        if g.dtype != spec.out_dtype:
            g = g.to(spec.out_dtype)
        if g.ndim != 2 or g.stride(-1) != 1:
            g = g.reshape(-1, dim).contiguous()
        keep.append(g)
        feats["out"][f] = g.data_ptr()
        feats["out_stride"][f] = g.stride(0)
        feats["weight"][f] = d.data_ptr()
        sel.append(f)
    if not sel:
        return
    sub = np.ascontiguousarray(feats[sel])
    target = forward_target_ids(sub)
    n_chunks = lib().mdl_plan_chunks(sub.ctypes.data, len(sub), target, None, 0)
    if n_chunks < 0:
        check(int(n_chunks), "mdl_plan_chunks")
    chunks = np.zeros(max(n_chunks, 1), dtype=CHUNK_DTYPE)
    lib().mdl_plan_chunks(sub.ctypes.data, len(sub), target, chunks.ctypes.data, n_chunks)
    device = res.device
    sub_dev = upload(sub, device)
    chunks_dev = upload(chunks, device)
    ids_arg = res.ids if res.ids.numel() else res.keep[-1]
    check(
        lib().mdl_pool_backward(
            sub_dev.data_ptr(), len(sub), chunks_dev.data_ptr(), n_chunks, ids_arg.data_ptr(), res.ids.numel(),
            res.offsets.data_ptr(), res.bag_count.data_ptr(), feature_classes(sub), _stream(device),
        ),
        "mdl_pool_backward",
    )
    del keep


def _segments(res: ForwardResult, feats: np.ndarray) -> list[tuple[KeyGroup, np.ndarray, int, int]]:
    """(key group, its backward descriptors, its first key, its key count) of
    each key group of a forward: a group's features are consecutive, so its
    keys are one stretch of the forward's key array."""

    groups = res.plan.groups
    if len(groups) == 1:
        return [(groups[0], feats, 0, res.num_ids)]
    out = []
    for g in groups:
        fs = np.ascontiguousarray(feats[g.lo: g.hi])
        first = int(fs["ids_begin"][0]) if len(fs) else 0
        out.append((g, fs, first, int(fs["num_ids"].sum())))
    return out


def backward_adagrad(
    res: ForwardResult,
    grads: Sequence[Tensor | None],
    *,
    lr: float,
    eps: float,
    clip_norm: float | None = None,
) -> Tensor | None:
    """Fused backward + row-wise Adagrad of every table (consumes the keys).

    With ``clip_norm`` the coalesced gradient of all tables is first clipped to
    that global 2-norm (the trainer's sparse clip, src/train.py:5788-5826)
    without being materialised; returns the pre-clip norm (device fp32 [1]).
    """

    plan = res.plan
    if res.keys is None:
        raise RuntimeError("the forward ran without backward bookkeeping")
    for t in plan.tables:
        if t.state is None:
            raise RuntimeError("every table needs a row-wise Adagrad accumulator")
    feats, keep = _attach_grads(res, grads)
    device = res.device
    stream = _stream(device)
    segs = []
    for g, fs, first, n in _segments(res, feats):
        tables = _tables_array(g.plan, fs)
        feats_dev = _CACHE.get(fs, device)
        tables_dev = _CACHE.get(tables, device)
        keep += [feats_dev, tables_dev]
        args = (feats_dev.data_ptr(), len(fs), tables_dev.data_ptr(), len(tables), plan.max_dim,
                res.keys.data_ptr() + 4 * first, res.payload.data_ptr() + 4 * first, n, plan.key_bits,
                _ptr(res.bag_count))
        segs.append((args, n, len(tables), table_classes(tables)))
    norm = None
    if clip_norm is None:
        # one workspace: each call sorts and reduces before the next one starts
        ws = _workspace(max(lib().mdl_backward_workspace_bytes(n, T, plan.max_dim) for _, n, T, _ in segs), device)
        for args, n, T, classes in segs:
            check(
                lib().mdl_backward_adagrad(*args[:8], None, *args[8:], float(lr), float(eps), None, ws.data_ptr(),
                                           ws.numel(), classes, stream),
                "mdl_backward_adagrad",
            )
    else:
        sumsq = torch.empty(len(segs), dtype=torch.float32, device=device)
        wss = []
        for i, (args, n, T, classes) in enumerate(segs):
            ws = _workspace(lib().mdl_backward_workspace_bytes(n, T, plan.max_dim), device)
            wss.append(ws)
            check(
                lib().mdl_backward_sort(args[2], T, plan.max_dim, args[5], args[6], n, None, plan.key_bits,
                                        ws.data_ptr(), ws.numel(), stream),
                "mdl_backward_sort",
            )
            check(lib().mdl_backward_sumsq(*args, sumsq.data_ptr() + 4 * i, ws.data_ptr(), ws.numel(), classes,
                                           stream),
                  "mdl_backward_sumsq")
        norm, coef = clip_coefficient(sumsq, clip_norm)
        for (args, n, T, classes), ws in zip(segs, wss):
            check(
                lib().mdl_backward_apply(*args, float(lr), float(eps), coef.data_ptr(), ws.data_ptr(), ws.numel(),
                                         classes, stream),
                "mdl_backward_apply",
            )
    res.keys = None
    res.payload = None
    del keep
    return norm


# ------------------------------------------------------------- clipping --


def _spans(tensors: Sequence[Tensor], live_rows: Sequence[Tensor | None] | None = None
           ) -> tuple[np.ndarray, list[Tensor]]:
    """Span descriptors of contiguous gradients; ``live_rows[i]`` (a device
    int64 [1], or None) limits span i to its first rows."""

    spans = np.zeros(len(tensors), dtype=_lib.SPAN_DTYPE)
    keep = list(tensors)
    for i, t in enumerate(tensors):
        _require_device(t, "gradient")
        if not t.is_contiguous():
            raise ValueError("gradients to clip must be contiguous")
        spans[i]["data"] = t.data_ptr()
        spans[i]["numel"] = t.numel()
        spans[i]["dtype"] = dtype_code(t.dtype)
        live = live_rows[i] if live_rows is not None else None
        if live is not None:
            if live.dtype != torch.int64 or live.device != t.device:
                raise ValueError("live row counts are int64 tensors on the gradient's device")
            spans[i]["row_elems"] = int(t[0].numel()) if t.dim() > 1 else 1
            spans[i]["live_rows"] = live.data_ptr()
            keep.append(live)
    return spans, keep


def grad_sumsq(tensors: Sequence[Tensor], device: torch.device,
               live_rows: Sequence[Tensor | None] | None = None) -> Tensor:
    """Sum of squares of every element of every tensor: fp32 [1] on device
    (of tensor i's first ``live_rows[i]`` rows only, when given)."""

    out = torch.empty(1, dtype=torch.float32, device=device)
    pairs = [(t, None if live_rows is None else live_rows[i]) for i, t in enumerate(tensors) if t.numel()]
    spans, _ = _spans([t for t, _ in pairs], [c for _, c in pairs])
    ws = _workspace(lib().mdl_sumsq_workspace_bytes(len(spans)), device)
    spans_dev = upload(spans, device) if len(spans) else None
    check(
        lib().mdl_sumsq(_ptr(spans_dev), len(spans), out.data_ptr(), ws.data_ptr(), ws.numel(), _stream(device)),
        "mdl_sumsq",
    )
    return out


def clip_coefficient(sumsq: Tensor, max_norm: float) -> tuple[Tensor, Tensor]:
    """(total norm, min(max_norm / (norm + 1e-6), 1)) from squared norms."""

    sumsq = sumsq.reshape(-1).to(torch.float32).contiguous()
    norm = torch.empty(1, dtype=torch.float32, device=sumsq.device)
    coef = torch.empty(1, dtype=torch.float32, device=sumsq.device)
    check(
        lib().mdl_clip_coef(sumsq.data_ptr(), sumsq.numel(), float(max_norm), norm.data_ptr(), coef.data_ptr(),
                            _stream(sumsq.device)),
        "mdl_clip_coef",
    )
    return norm, coef


def scale_(tensors: Sequence[Tensor], coef: Tensor, live_rows: Sequence[Tensor | None] | None = None) -> None:
    """In-place ``t *= coef`` in each tensor's dtype (coef: device fp32 [1]);
    of tensor i's first ``live_rows[i]`` rows only, when given."""

    pairs = [(t, None if live_rows is None else live_rows[i]) for i, t in enumerate(tensors) if t.numel()]
    if not pairs:
        return
    spans, _ = _spans([t for t, _ in pairs], [c for _, c in pairs])
    device = pairs[0][0].device
    spans_dev = upload(spans, device)
    check(lib().mdl_scale(spans_dev.data_ptr(), len(spans), coef.data_ptr(), _stream(device)), "mdl_scale")


def backward_coalesce(res: ForwardResult, grads: Sequence[Tensor | None]) -> list[tuple[Tensor, Tensor]]:
    """Coalesced sparse gradient ``(rows, values)`` of every table.

    Rows are ascending and unique; values have the table's dtype.  Syncs once
    (to size the per-table outputs).
    """

    plan = res.plan
    if res.keys is None:
        raise RuntimeError("the forward ran without backward bookkeeping")
    feats, keep = _attach_grads(res, grads)
    device = res.device
    stream = _stream(device)
    T = len(plan.tables)
    segs = []
    ranges = []
    for g, fs, first, n in _segments(res, feats):
        tables = _tables_array(g.plan, fs)
        feats_dev = upload(fs, device)
        tables_dev = upload(tables, device)
        Tg = len(tables)
        ws = _workspace(lib().mdl_backward_workspace_bytes(n, Tg, plan.max_dim), device)
        urange = torch.zeros(2 * Tg, dtype=torch.int64, device=device)
        keys, payload = res.keys.data_ptr() + 4 * first, res.payload.data_ptr() + 4 * first
        check(
            lib().mdl_backward_count(
                tables_dev.data_ptr(), Tg, plan.max_dim, keys, payload, n, None, plan.key_bits, urange.data_ptr(),
                ws.data_ptr(), ws.numel(), stream,
            ),
            "mdl_backward_count",
        )
        segs.append((g, fs, feats_dev, tables, tables_dev, ws, urange, keys, payload, n))
        ranges.append(urange)
    ur_host = torch.cat(ranges).cpu().numpy().reshape(-1, 2)
    us = np.zeros(T, dtype=np.int64)
    k = 0
    for g, *_ in segs:
        us[g.tables] = ur_host[k: k + len(g.tables), 1] - ur_host[k: k + len(g.tables), 0]
        k += len(g.tables)
    # Two allocations for all tables, the rows split per table and the values
    # as per-table views of one byte buffer, each starting on a 256-byte
    # boundary (the kernel stores 16-byte vectors).  The kernel's output
    # addresses come from the two bases, so it is launched before the 200-odd
    # per-table views are built on the host (that loop overlaps the GPU).
    esz = np.array([t.weight.element_size() for t in plan.tables], dtype=np.int64)
    dims = np.array([int(t.weight.size(1)) for t in plan.tables], dtype=np.int64)
    nbytes = us * dims * esz
    offs = np.zeros(T + 1, dtype=np.int64)
    np.cumsum((nbytes + 255) // 256 * 256, out=offs[1:])
    rows_off = np.zeros(T + 1, dtype=np.int64)
    np.cumsum(us, out=rows_off[1:])
    rows_all = torch.empty(int(rows_off[-1]), dtype=torch.int64, device=device)
    vbuf = torch.empty(int(offs[-1]), dtype=torch.uint8, device=device)
    for g, fs, feats_dev, tables, tables_dev, ws, urange, keys, payload, n in segs:
        if not n:
            continue
        tg = np.asarray(g.tables, dtype=np.int64)
        Tg = len(tg)
        addr = np.zeros(2 * Tg, dtype=np.uint64)
        addr[:Tg] = np.where(us[tg] > 0, rows_all.data_ptr() + 8 * rows_off[tg], 0).astype(np.uint64)
        addr[Tg:] = np.where(us[tg] > 0, vbuf.data_ptr() + offs[tg], 0).astype(np.uint64)
        addr_dev = upload(addr, device)
        keep.append(addr_dev)
        check(
            lib().mdl_backward_coalesce(
                feats_dev.data_ptr(), len(fs), tables_dev.data_ptr(), Tg, plan.max_dim, keys, payload, n,
                plan.key_bits, _ptr(res.bag_count), urange.data_ptr(), addr_dev.data_ptr(),
                addr_dev.data_ptr() + 8 * Tg, ws.data_ptr(), ws.numel(), table_classes(tables), stream,
            ),
            "mdl_backward_coalesce",
        )
    rows_list = rows_all.split(us.tolist())
    result = []
    for t, table in enumerate(plan.tables):
        w = table.weight
        vals = vbuf[int(offs[t]): int(offs[t]) + int(nbytes[t])].view(w.dtype).view(int(us[t]), int(dims[t]))
        result.append((rows_list[t], vals))
    res.keys = None
    res.payload = None
    del keep
    return result


def table_capacities(res: ForwardResult) -> np.ndarray:
    """Ids looked up on each table by this forward (host-known from the
    shapes): a bound on its distinct rows."""

    cap = np.zeros(len(res.plan.tables), dtype=np.int64)
    np.add.at(cap, np.asarray(res.feats["table"], dtype=np.int64), np.asarray(res.feats["num_ids"], dtype=np.int64))
    return cap


def coalesced_layout(weights: Sequence[Tensor], cap: Sequence[int], memo: dict | None = None) -> dict:
    """Where capacity-sized coalesced gradients live in two flat buffers:
    rows of table t at ``rows_off[t]`` (int64 elements), values at byte
    ``val_off[t]`` (each table's region 256-byte aligned).  ``memo``: a
    layout's memo holding its tables' element sizes and dims."""

    cap = np.asarray(cap, dtype=np.int64)
    T = len(weights)
    sizes = memo.get("esz_dims") if memo is not None else None
    if sizes is None:
        sizes = (np.array([w.element_size() for w in weights], dtype=np.int64),
                 np.array([int(w.size(1)) for w in weights], dtype=np.int64))
        if memo is not None:
            memo["esz_dims"] = sizes
    esz, dims = sizes
    nbytes = cap * dims * esz
    val_off = np.zeros(T + 1, dtype=np.int64)
    np.cumsum((nbytes + 255) // 256 * 256, out=val_off[1:])
    rows_off = np.zeros(T + 1, dtype=np.int64)
    np.cumsum(cap, out=rows_off[1:])
    return {"cap": cap, "dims": dims, "nbytes": nbytes, "val_off": val_off, "rows_off": rows_off}


def split_coalesced(weights: Sequence[Tensor], rows_all: Tensor, vbuf: Tensor, layout: dict
                    ) -> tuple[list[Tensor], list[Tensor]]:
    """Per-table ``rows [cap_t]`` and ``values [cap_t, dim]`` views."""

    cap, dims, nbytes, val_off = layout["cap"], layout["dims"], layout["nbytes"], layout["val_off"]
    rows = list(rows_all[: int(layout["rows_off"][-1])].split(cap.tolist()))
    values = [vbuf[int(val_off[t]): int(val_off[t]) + int(nbytes[t])].view(w.dtype).view(int(cap[t]), int(dims[t]))
              for t, w in enumerate(weights)]
    return rows, values


def backward_coalesce_padded(
    res: ForwardResult, grads: Sequence[Tensor | None]
) -> tuple[Tensor, Tensor, Tensor, dict]:
    """Coalesced sparse gradient of every table without a host read.

    Table t gets ``cap_t`` entries (its id count): the first ``counts[t]`` are
    the coalesced gradient (rows ascending, unique), the rest repeat the last
    row with zero values, so each table's pair is a valid uncoalesced COO
    gradient with the same sum.  Returns ``(rows_all, values_bytes, counts,
    layout)``: two flat buffers (see :func:`coalesced_layout`,
    :func:`split_coalesced`) and ``counts``, a device int64 ``[T]``.  Only
    launches.
    """

    plan = res.plan
    if res.keys is None:
        raise RuntimeError("the forward ran without backward bookkeeping")
    feats, keep = _attach_grads(res, grads)
    device = res.device
    T = len(plan.tables)
    stream = _stream(device)
    cap = table_capacities(res)
    layout = coalesced_layout([t.weight for t in plan.tables], cap, memo=plan._memo)
    rows_off, val_off = layout["rows_off"], layout["val_off"]
    rows_all = torch.empty(max(int(rows_off[-1]), 1), dtype=torch.int64, device=device)
    vbuf = torch.empty(max(int(val_off[-1]), 1), dtype=torch.uint8, device=device)
    segs = _segments(res, feats)
    urange = torch.zeros(2 * sum(len(g.tables) for g, *_ in segs), dtype=torch.int64, device=device)
    ws = None
    u0 = 0
    for g, fs, first, n in segs:
        Tg = len(g.tables)
        ur = urange.data_ptr() + 8 * u0
        u0 += 2 * Tg
        if not n:
            continue
        tg = np.asarray(g.tables, dtype=np.int64)
        cg = cap[tg]
        pad_units = (cg + 63) // 64
        unit_first = np.zeros(Tg + 1, dtype=np.int64)
        np.cumsum(pad_units, out=unit_first[1:])
        # one upload: row and value addresses, capacities, pad-unit prefix
        host = np.concatenate([
            np.where(cg > 0, rows_all.data_ptr() + 8 * rows_off[tg], 0).astype(np.uint64).view(np.int64),
            np.where(cg > 0, vbuf.data_ptr() + val_off[tg], 0).astype(np.uint64).view(np.int64),
            cg, unit_first,
        ])
        meta = upload(host, device)
        base = meta.data_ptr()
        tables = _tables_array(g.plan, fs)
        feats_dev = _CACHE.get(fs, device)
        tables_dev = _CACHE.get(tables, device)
        keep += [meta, feats_dev, tables_dev]
        # one workspace: each group's calls finish before the next group's
        need = lib().mdl_backward_workspace_bytes(n, Tg, plan.max_dim)
        if ws is None or ws.numel() < need:
            ws = _workspace(need, device)
            keep.append(ws)
        keys, payload = res.keys.data_ptr() + 4 * first, res.payload.data_ptr() + 4 * first
        check(
            lib().mdl_backward_count(
                tables_dev.data_ptr(), Tg, plan.max_dim, keys, payload, n, None, plan.key_bits, ur, ws.data_ptr(),
                ws.numel(), stream,
            ),
            "mdl_backward_count",
        )
        check(
            lib().mdl_backward_coalesce(
                feats_dev.data_ptr(), len(fs), tables_dev.data_ptr(), Tg, plan.max_dim, keys, payload, n,
                plan.key_bits, _ptr(res.bag_count), ur, base, base + 8 * Tg, ws.data_ptr(), ws.numel(),
                table_classes(tables), stream,
            ),
            "mdl_backward_coalesce",
        )
        check(
            lib().mdl_backward_pad(
                tables_dev.data_ptr(), Tg, ur, base, base + 8 * Tg, base + 16 * Tg, base + 24 * Tg,
                int(unit_first[-1]), stream,
            ),
            "mdl_backward_pad",
        )
    if len(segs) == 1 and segs[0][0].tables == list(range(T)):
        counts = urange[1::2] - urange[0::2]
    else:
        order = np.concatenate([np.asarray(g.tables, dtype=np.int64) for g, *_ in segs])
        counts = torch.zeros(T, dtype=torch.int64, device=device)
        counts.index_copy_(0, upload(order, device).view(torch.int64), urange[1::2] - urange[0::2])
    res.keys = None
    res.payload = None
    del keep
    return rows_all, vbuf, counts, layout


def grouped_rowwise_adagrad_(
    weights: Sequence[Tensor],
    accumulators: Sequence[Tensor],
    rows: Sequence[Tensor],
    values: Sequence[Tensor],
    counts: Sequence[Tensor | None],
    lrs: Sequence[float],
    *,
    eps: float,
    error_count: Tensor | None = None,
) -> None:
    """Row-wise Adagrad of many tables in one launch (src/optim.py:299-377).

    Table i updates rows[i][:n] with values[i][:n], n read on the device from
    ``counts[i]`` (an int64 element; None: all rows).  Rows must be unique.
    """

    if not weights:
        return
    device = weights[0].device
    rows = list(rows)
    values = list(values)
    for i, (w, a, r, v) in enumerate(zip(weights, accumulators, rows, values)):
        if w.device.type != "cuda":
            _require_device(w, "weight")
        if w.ndim != 2 or w.stride(1) != 1:
            raise ValueError("row-wise Adagrad expects 2D weights with contiguous rows")
        if a.dtype != torch.float32 or not a.is_contiguous():
            raise TypeError("row-wise Adagrad accumulator must be a contiguous float32 tensor")
        if r.dtype != torch.int64 or not r.is_contiguous():
            rows[i] = r.to(torch.int64).contiguous()
        if (w.dtype == torch.float32 and v.dtype != torch.float32) or v.dtype not in (torch.float32, torch.bfloat16):
            v = values[i] = v.float()
        if not v.is_contiguous() or v.data_ptr() % 16:
            values[i] = _row_major_aligned(v)
    keep = rows + values
    ups = np.zeros(len(weights), dtype=_lib.UPDATE_DTYPE)
    ups["weight"] = [w.data_ptr() for w in weights]
    ups["state"] = [a.data_ptr() for a in accumulators]
    ups["rows"] = [r.data_ptr() for r in rows]
    ups["values"] = [v.data_ptr() for v in values]
    ups["count"] = [0 if c is None else c.data_ptr() for c in counts]
    shapes = [w.shape for w in weights]
    ups["num_rows"] = [sh[0] for sh in shapes]
    ups["dim"] = [sh[1] for sh in shapes]
    ups["capacity"] = [r.numel() for r in rows]
    ups["weight_stride"] = [w.stride(0) for w in weights]
    ups["values_stride"] = [v.stride(0) if v.ndim == 2 and v.size(0) else sh[1] for v, sh in zip(values, shapes)]
    ups["wdtype"] = [dtype_code(w.dtype) for w in weights]
    ups["vdtype"] = [dtype_code(v.dtype) for v in values]
    ups["lr"] = np.asarray(lrs, dtype=np.float32)
    units = (ups["capacity"] + _lib.MDL_UPDATE_UNIT - 1) // _lib.MDL_UPDATE_UNIT
    ups["unit_first"][1:] = np.cumsum(units)[:-1]
    if int(units.sum()) == 0:
        return
    ups_dev = upload(ups, device)
    check(
        lib().mdl_grouped_rowwise_adagrad(ups_dev.data_ptr(), ups.ctypes.data, len(ups), float(eps),
                                          _ptr(error_count), _stream(device)),
        "mdl_grouped_rowwise_adagrad",
    )
    del keep


def coalesce_rows(
    indices: Tensor, values: Tensor, num_rows: int, *, padding_idx: int = -1
) -> tuple[Tensor, Tensor]:
    """Sort + unique + segment-sum of an uncoalesced COO gradient.

    ``indices`` [n] row ids, ``values`` [n, dim]; returns ``(rows, summed)``
    with rows ascending and unique (the work ``Tensor.coalesce()`` does for
    src/optim.py:323-324).  Syncs once.
    """

    _require_device(values, "values")
    device = values.device
    n = int(indices.numel())
    dim = int(values.size(1))
    if n == 0:
        return indices.new_empty(0), values.new_empty((0, dim))
    indices = indices.to(torch.int64).contiguous()
    values = _row_major_aligned(values)
    plan = GroupPlan()
    # A stand-in table of the right shape: only its row count, dim and dtype
    # are read, never its rows.
    fake_w = torch.empty((0, dim), dtype=values.dtype, device=device)
    plan.tables.append(TableSpec(weight=fake_w, state=None, row_base=0))
    plan.total_rows = int(num_rows)
    plan.features.append(FeatureSpec(table=0, pooling=MDL_POOL_NONE, exclude_null=False,
                                     padding_idx=padding_idx, out_dtype=values.dtype))
    keys = torch.empty(n, dtype=torch.int32, device=device)
    payload = torch.empty(n, dtype=torch.int32, device=device)
    err = torch.zeros(1, dtype=torch.int32, device=device)
    stream = _stream(device)
    check(
        lib().mdl_sparse_keys(
            indices.data_ptr(), n, int(num_rows), 0, 0, int(padding_idx), keys.data_ptr(),
            payload.data_ptr(), plan.sentinel, err.data_ptr(), stream,
        ),
        "mdl_sparse_keys",
    )
    feats = np.zeros(1, dtype=FEATURE_DTYPE)
    rec = feats[0]
    rec["grad"] = values.data_ptr()
    rec["num_rows"] = int(num_rows)
    rec["out_stride"] = values.stride(0)
    rec["num_ids"] = n
    rec["dim"] = dim
    rec["wdtype"] = dtype_code(values.dtype)
    rec["odtype"] = dtype_code(values.dtype)
    rec["pooling"] = MDL_POOL_NONE
    rec["padding_idx"] = padding_idx
    tables = np.zeros(1, dtype=TABLE_DTYPE)
    tables[0]["num_rows"] = int(num_rows)
    tables[0]["dim"] = dim
    tables[0]["wdtype"] = dtype_code(values.dtype)
    tables[0]["feature"] = 0
    tables[0]["gdtype"] = dtype_code(values.dtype)
    res = ForwardResult(
        plan=plan, device=device, ids=indices, offsets=None, outputs=[values], feats=feats,
        keys=keys, payload=payload, bag_count=None, error_count=err,
    )
    feats_dev = upload(feats, device)
    tables_dev = upload(tables, device)
    ws = _workspace(lib().mdl_backward_workspace_bytes(n, 1, dim), device)
    urange = torch.zeros(2, dtype=torch.int64, device=device)
    check(
        lib().mdl_backward_count(
            tables_dev.data_ptr(), 1, dim, keys.data_ptr(), payload.data_ptr(), n, None, plan.key_bits,
            urange.data_ptr(), ws.data_ptr(), ws.numel(), stream,
        ),
        "mdl_backward_count",
    )
    if int(err.item()):
        raise IndexError(f"sparse gradient rows outside [0, {num_rows})")
    u = int((urange[1] - urange[0]).item())
    rows = torch.empty(u, dtype=torch.int64, device=device)
    summed = torch.empty((u, dim), dtype=values.dtype, device=device)
    if u:
        rows_dev = upload(np.array([rows.data_ptr()], dtype=np.uint64), device)
        vals_dev = upload(np.array([summed.data_ptr()], dtype=np.uint64), device)
        check(
            lib().mdl_backward_coalesce(
                feats_dev.data_ptr(), 1, tables_dev.data_ptr(), 1, dim, keys.data_ptr(), payload.data_ptr(),
                n, plan.key_bits, None, urange.data_ptr(), rows_dev.data_ptr(), vals_dev.data_ptr(),
                ws.data_ptr(), ws.numel(), table_classes(tables), stream,
            ),
            "mdl_backward_coalesce",
        )
    del res
    return rows, summed


# ------------------------------------------------------------- sequences --


def sequence_forward(
    weight: Tensor,
    ids: Tensor,
    lengths: Tensor,
    *,
    out_len: int | None = None,
    order: str = "oldest_to_newest",
    padding_idx: int = 0,
    out_dtype: torch.dtype | None = None,
    keys: Tensor | None = None,
    payload: Tensor | None = None,
    row_base: int = 0,
    payload_base: int = 0,
    sentinel: int = 0,
    error_count: Tensor | None = None,
) -> tuple[Tensor, Tensor]:
    """Right-aligned sequence gather: ``([B, L, dim] embeddings, [B, L] mask)``.

    Semantics of F.embedding + ``_right_aligned_sequence`` (+ the reversal
    of ``_align_sequence_inputs`` for newest_to_oldest), src/model.py:2989-3100.
    """

    _require_device(ids, "sequence ids")
    if ids.dtype != torch.long:
        raise TypeError("sharded embedding indices must be torch.long")
    if ids.ndim != 2:
        raise ValueError("sequence ids must be [batch, length]")
    batch, in_len = int(ids.size(0)), int(ids.size(1))
    out_len = in_len if out_len is None else int(out_len)
    device = ids.device
    out_dtype = out_dtype or weight.dtype
    dim = int(weight.size(1))
    out = torch.empty((batch, out_len, dim), dtype=out_dtype, device=device)
    mask = torch.empty((batch, out_len), dtype=torch.bool, device=device)
    feat = np.zeros(1, dtype=FEATURE_DTYPE)
    rec = feat[0]
    rec["weight"] = weight.data_ptr()
    rec["num_rows"] = int(weight.size(0))
    rec["row_base"] = row_base
    rec["payload_base"] = payload_base
    rec["dim"] = dim
    rec["wdtype"] = dtype_code(weight.dtype)
    rec["odtype"] = dtype_code(out_dtype)
    rec["padding_idx"] = padding_idx
    order_code = _lib.MDL_SEQ_OLDEST_TO_NEWEST if order == "oldest_to_newest" else _lib.MDL_SEQ_NEWEST_TO_OLDEST
    if order not in ("oldest_to_newest", "newest_to_oldest"):
        raise ValueError("order must be oldest_to_newest or newest_to_oldest")
    ids = ids.contiguous()
    lengths = lengths.to(device=device, dtype=torch.int64).contiguous()
    check(
        lib().mdl_sequence_forward(
            feat.ctypes.data, ids.data_ptr(), lengths.data_ptr(), batch, in_len, out_len, order_code,
            out.data_ptr(), mask.data_ptr(), _ptr(keys), _ptr(payload), None, int(sentinel), _ptr(error_count),
            _stream(device),
        ),
        "mdl_sequence_forward",
    )
    return out, mask


def sequence_feature(
    weight: Tensor,
    *,
    state: Tensor | None = None,
    padding_idx: int = 0,
    out_dtype: torch.dtype | None = None,
    row_base: int = 0,
    payload_base: int = 0,
    grad: Tensor | None = None,
) -> np.ndarray:
    """Descriptor of one sequence feature: an unpooled feature whose output
    rows are the ``[B * out_len]`` positions of the padded window."""

    feat = np.zeros(1, dtype=FEATURE_DTYPE)
    rec = feat[0]
    rec["weight"] = weight.data_ptr()
    rec["state"] = state.data_ptr() if state is not None else 0
    rec["grad"] = grad.data_ptr() if grad is not None else 0
    rec["num_rows"] = int(weight.size(0))
    rec["out_stride"] = int(weight.size(1))
    rec["row_base"] = row_base
    rec["payload_base"] = payload_base
    rec["dim"] = int(weight.size(1))
    rec["wdtype"] = dtype_code(weight.dtype)
    rec["odtype"] = dtype_code(out_dtype or weight.dtype)
    rec["pooling"] = MDL_POOL_NONE
    rec["padding_idx"] = padding_idx
    return feat


def sequence_lookup(
    weight: Tensor,
    ids: Tensor,
    lengths: Tensor,
    *,
    out_len: int | None = None,
    order: str = "oldest_to_newest",
    padding_idx: int = 0,
    with_backward: bool = True,
    error_count: Tensor | None = None,
) -> ForwardResult:
    """Right-aligned sequence gather with backward bookkeeping.

    ``outputs[0]`` is ``[B, out_len, dim]`` and ``keep[0]`` the ``[B, out_len]``
    mask; the result feeds :func:`backward_coalesce` like a grouped lookup.
    """

    plan = GroupPlan()
    plan.add_feature(weight, pooling="none", padding_idx=padding_idx)
    device = ids.device
    if ids.ndim != 2:
        raise ValueError("sequence ids must be [batch, length]")
    # one sort entry per window position
    n = int(ids.size(0)) * int(ids.size(1) if out_len is None else out_len)
    keys = payload = None
    if with_backward:
        keys = torch.empty(max(n, 1), dtype=torch.int32, device=device)
        payload = torch.empty(max(n, 1), dtype=torch.int32, device=device)
    if error_count is None:
        error_count = torch.zeros(1, dtype=torch.int32, device=device)
    out, mask = sequence_forward(
        weight, ids, lengths, out_len=out_len, order=order, padding_idx=padding_idx, keys=keys,
        payload=payload, row_base=0, payload_base=0, sentinel=plan.sentinel, error_count=error_count,
    )
    feats = sequence_feature(weight, padding_idx=padding_idx)
    return ForwardResult(
        plan=plan, device=device, ids=ids, offsets=None, outputs=[out], feats=feats, keys=keys,
        payload=payload, bag_count=None, error_count=error_count, keep=[mask], count=n,
    )
