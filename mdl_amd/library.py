"""The sparse path as torch.library custom ops, namespace ``mdl_hip``.

Each op has one schema and three implementations:

* ROCm devices: the hand-written gfx950 kernels of libmdl_hip.so, through
  its C ABI (``mdl_amd.ops``);
* CPU: PyTorch CPU operations with the reference's CPU semantics, so
  modules whose parameters live on the CPU work as in the reference
  (src/embeddings.py:468-473, src/model.py:509-678, src/optim.py:359-376);
* fake tensors: shapes only, for tracing and ``torch.compile``.

Ops:

``mdl_hip::bucketize``                 pre_hashed / mod bucketing (src/features.py:360-376, src/benchmark.py:1246-1250)
``mdl_hip::lengths_to_offsets``        CSR offsets of bag lengths
``mdl_hip::grouped_lookup``            grouped lookup + sum/mean bag pooling (src/embeddings.py:1646-1709, src/model.py:509-678)
``mdl_hip::grouped_lookup_backward``   its coalesced sparse weight gradients, capacity-sized (no host read)
``mdl_hip::sequence_lookup``           right-aligned sequence window gather (src/model.py:2989-3100)
``mdl_hip::sequence_lookup_backward``  its coalesced sparse weight gradient, capacity-sized
``mdl_hip::sparse_coalesce``           sort + unique + segment sum of a COO gradient (src/optim.py:321-324)
``mdl_hip::sparse_coalesce_padded``    the same, capacity-sized (no host read)
``mdl_hip::rowwise_adagrad_``          row-wise Adagrad of one table (src/optim.py:68-108, CPU :359-376)
``mdl_hip::grouped_rowwise_adagrad_``  row-wise Adagrad of many tables in one launch, row counts read on device

Capacity-sized gradients: table t's gradient has ``cap_t`` entries (its id
count, a bound on its distinct rows that the host knows from the shapes);
the first ``counts[t]`` are the coalesced rows (ascending, unique) and the
rest repeat the last row with zero values.  The pair is a valid uncoalesced
COO gradient with the coalesced sum, and its size needs no device-to-host
read; ``grouped_rowwise_adagrad_`` reads ``counts`` on the device.
"""

from __future__ import annotations

import weakref
from collections import OrderedDict
from typing import Optional

import numpy as np
import torch
from torch import Tensor

from . import _lib, ops

_POOL = {0: "none", 1: "sum", 2: "mean"}
_CUDA = "cuda"


def _is_rocm(t: Tensor) -> bool:
    return t.device.type == _CUDA


# ------------------------------------------------------------- bucketing --


@torch.library.custom_op("mdl_hip::bucketize", mutates_args=(), device_types=_CUDA)
def bucketize(raw: Tensor, valid: Optional[Tensor], num_buckets: int, mode: str,
              validate_nonzero: bool) -> tuple[Tensor, Tensor]:
    err = torch.zeros(1, dtype=torch.int32, device=raw.device)
    out = ops.bucketize(raw, num_buckets, mode=mode, valid=valid, validate_nonzero=validate_nonzero,
                        error_count=err)
    return out, err


@bucketize.register_kernel("cpu")
def _bucketize_cpu(raw, valid, num_buckets, mode, validate_nonzero):
    if raw.dtype != torch.int64:
        raise TypeError("raw ids must be torch.int64")
    if mode == "pre_hashed":
        if num_buckets <= 0 or num_buckets & (num_buckets - 1):
            raise ValueError("pre_hashed num_buckets must be a power of two")
        # two's complement & (B - 1) is the uint64 mask for B <= 2^62
        out = (raw & (num_buckets - 1)) + 1
        zeros = raw == 0
    elif mode == "mod":
        if num_buckets <= 1:
            raise ValueError("mod bucketing needs num_buckets > 1")
        m = num_buckets - 1
        r = torch.remainder(raw, m)  # floor-mod, no overflow at INT64_MIN
        out = torch.where(r == 0, m, r)  # 1 + floormod(raw - 1, m)
        zeros = torch.zeros_like(raw, dtype=torch.bool)
    else:
        raise ValueError("mode must be pre_hashed or mod")
    if valid is not None:
        v = valid.to(torch.bool)
        out = torch.where(v, out, 0)
        zeros = zeros & v
    count = int(zeros.sum()) if (validate_nonzero and mode == "pre_hashed") else 0
    return out, torch.tensor([count], dtype=torch.int32)


@bucketize.register_fake
def _bucketize_fake(raw, valid, num_buckets, mode, validate_nonzero):
    return torch.empty_like(raw), raw.new_empty(1, dtype=torch.int32)


def _bucket_values_cpu(raw: Tensor, present: Tensor, num_buckets: int, mode: str,
                       validate_nonzero: bool) -> tuple[Tensor, int]:
    """Ids of raw values (0 for nulls) and the count of non-null zeros under
    a validated pre_hashed rule."""

    if mode == "none":
        return torch.where(present, raw, 0), 0
    out, err = _bucketize_cpu(raw, present.to(torch.uint8), num_buckets, mode, validate_nonzero)
    return out, int(err[0])


@torch.library.custom_op("mdl_hip::bag_truncate", mutates_args=(), device_types=_CUDA)
def bag_truncate(values: Tensor, offsets: Tensor, valid: Optional[Tensor], row_valid: Optional[Tensor],
                 max_length: int, truncation: str, bucket: str, num_buckets: int,
                 validate_nonzero: bool) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """List feature -> CSR bag: ``(ids [n_in], lengths [rows], offsets
    [rows+1], error count [1])``; ids past the kept total (``offsets[-1]``)
    are 0.  ``max_length < 0``: no truncation.  The error count adds rows
    whose offsets fall outside the values (clamped) and non-null zeros under
    a validated pre_hashed rule."""

    err = torch.zeros(1, dtype=torch.int32, device=values.device)
    ids, lengths, out_offsets = ops.bag_truncate(
        values, offsets, valid=valid, row_valid=row_valid, max_length=None if max_length < 0 else max_length,
        truncation=truncation, bucket=bucket, num_buckets=num_buckets, validate_nonzero=validate_nonzero,
        error_count=err)
    return ids, lengths, out_offsets, err


@bag_truncate.register_kernel("cpu")
def _bag_truncate_cpu(values, offsets, valid, row_valid, max_length, truncation, bucket, num_buckets,
                      validate_nonzero):
    if values.dtype != torch.int64 or offsets.dtype != torch.int64:
        raise TypeError("list values and offsets must be torch.int64")
    if truncation not in ops.TRUNCATIONS:
        raise ValueError(f"unsupported list truncation {truncation!r}")
    if bucket not in ops.BUCKET_MODES:
        raise ValueError(f"bucket must be one of {sorted(ops.BUCKET_MODES)}")
    n_in = int(values.numel())
    rows = int(offsets.numel()) - 1
    if rows < 0:
        raise ValueError("list offsets need at least one entry")
    lo_raw, hi_raw = offsets[:-1], offsets[1:]
    lo = lo_raw.clamp(0, n_in)
    hi = torch.maximum(hi_raw.clamp(max=n_in), lo)
    bad = int(((lo_raw < 0) | (lo_raw > n_in) | (hi_raw < lo) | (hi_raw > n_in)).sum())
    length = hi - lo
    if row_valid is not None and not (truncation == "tail" and max_length >= 0):
        # tail truncation reads every row's raw offsets (src/dataloader.py:8583-8604)
        length = torch.where(row_valid != 0, length, 0)
    take = length if max_length < 0 else length.clamp(max=max_length)
    starts = lo if truncation == "head" else hi - take
    total = int(take.sum())
    row_ids = torch.repeat_interleave(torch.arange(rows), take)
    within = torch.arange(total) - torch.repeat_interleave(torch.cumsum(take, 0) - take, take)
    src = starts[row_ids] + within
    present = valid[src] != 0 if valid is not None else torch.ones(total, dtype=torch.bool)
    kept, zeros = _bucket_values_cpu(values[src], present, num_buckets, bucket, validate_nonzero)
    ids = torch.zeros(n_in, dtype=torch.int64)
    ids[:total] = kept
    out_offsets = torch.zeros(rows + 1, dtype=torch.int64)
    torch.cumsum(take, 0, out=out_offsets[1:])
    return ids, take.clone(), out_offsets, torch.tensor([bad + zeros], dtype=torch.int32)


@bag_truncate.register_fake
def _bag_truncate_fake(values, offsets, valid, row_valid, max_length, truncation, bucket, num_buckets,
                       validate_nonzero):
    rows = offsets.size(0) - 1
    return (values.new_empty(values.size(0), dtype=torch.int64), offsets.new_empty(rows, dtype=torch.int64),
            offsets.new_empty(rows + 1, dtype=torch.int64), values.new_empty(1, dtype=torch.int32))


@torch.library.custom_op("mdl_hip::lengths_to_offsets", mutates_args=(), device_types=_CUDA)
def lengths_to_offsets(lengths: Tensor) -> Tensor:
    return ops.lengths_to_offsets(lengths)


@lengths_to_offsets.register_kernel("cpu")
def _offsets_cpu(lengths):
    out = torch.zeros(lengths.numel() + 1, dtype=torch.int64)
    torch.cumsum(lengths.to(torch.int64), 0, out=out[1:])
    return out


@lengths_to_offsets.register_fake
def _offsets_fake(lengths):
    return lengths.new_empty(lengths.numel() + 1, dtype=torch.int64)


# ------------------------------------------------------- grouped lookup --


def _layout(ids, lengths, pooling):
    """(ids per feature, output rows per feature, offsets entries, pooled?)."""

    pooled_any = any(p != 0 for p in pooling)
    n_ids = [int(x.numel()) for x in ids]
    rows_out = [int(ln.numel()) if p != 0 else n for ln, p, n in zip(lengths, pooling, n_ids)]
    n_len = sum(int(ln.numel()) if p != 0 else 1 for ln, p in zip(lengths, pooling)) if pooled_any else 0
    return n_ids, rows_out, n_len, pooled_any


def _check_features(weights, ids, lengths, table, pooling, exclude, padding_idx):
    nf = len(ids)
    if not (len(lengths) == len(table) == len(pooling) == len(exclude) == len(padding_idx) == nf):
        raise ValueError("one entry per feature in ids, lengths, table, pooling, exclude and padding_idx")
    for f in range(nf):
        if ids[f].dtype != torch.long:
            raise TypeError("sharded embedding indices must be torch.long")
        if not 0 <= table[f] < len(weights):
            raise ValueError("feature table index out of range")
        if pooling[f] not in _POOL:
            raise ValueError(f"unsupported pooling code {pooling[f]}")
        if pooling[f] != 0 and (lengths[f] is None or lengths[f].ndim != 1):
            raise ValueError("categorical bag lengths must have shape [B]")


def _order(weights, table) -> Optional[list[int]]:
    """Feature order of a device call: the callers' order, except that a call
    over 2^32 - 1 table rows or more looks its features up sorted by table, so
    that each key group's features are consecutive (its keys one stretch)."""

    if sum(int(w.size(0)) for w in weights) < ops.KEY_SPACE:
        return None
    order = sorted(range(len(table)), key=lambda f: table[f])
    return None if order == list(range(len(table))) else order


# Layouts seen by the device ops, most recent last: what a plan of the same
# weights (addresses, shapes, dtypes) and features derives on the host -- row
# bases, feature specs and the memo of descriptor columns -- so a training
# loop builds each layout's host arrays once.  Entries hold addresses and
# sizes, never tensors: a freed table keeps nothing alive, and a new table
# at the same address with the same shape and dtype is described the same.
_LAYOUTS: "OrderedDict[tuple, dict]" = OrderedDict()
_LAYOUTS_MAX = 16


def _plan(weights, table, pooling, exclude, padding_idx) -> ops.GroupPlan:
    key = (weights[0].device, tuple((w.data_ptr(), w.shape, w.dtype, w.stride(0)) for w in weights),
           tuple(table), tuple(pooling), tuple(exclude), tuple(padding_idx))
    entry = _LAYOUTS.get(key)
    if entry is None:
        plan = ops.GroupPlan()
        for w in weights:
            plan.add_table(w, None, shared=False)
        for f in range(len(table)):
            plan.features.append(ops.FeatureSpec(
                table=int(table[f]), pooling=int(pooling[f]), exclude_null=bool(exclude[f]),
                padding_idx=int(padding_idx[f]), out_dtype=weights[table[f]].dtype,
            ))
        entry = {"bases": [t.row_base for t in plan.tables], "total": plan.total_rows,
                 "features": plan.features, "memo": {}}
        _LAYOUTS[key] = entry
        if len(_LAYOUTS) > _LAYOUTS_MAX:
            _LAYOUTS.popitem(last=False)
    else:
        _LAYOUTS.move_to_end(key)
        plan = ops.GroupPlan()
        plan.tables = [ops.TableSpec(weight=w, state=None, row_base=b) for w, b in zip(weights, entry["bases"])]
        plan.features = entry["features"]
        plan.total_rows = entry["total"]
    plan._memo = entry["memo"]
    return plan


@torch.library.custom_op("mdl_hip::grouped_lookup", mutates_args=(), device_types=_CUDA)
def grouped_lookup(
    weights: list[Tensor], ids: list[Tensor], lengths: list[Optional[Tensor]], table: list[int],
    pooling: list[int], exclude: list[int], padding_idx: list[int], need_backward: bool,
) -> tuple[list[Tensor], Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Outputs per feature (``[*ids.shape, dim]`` unpooled, ``[B, dim]``
    pooled) and the backward's bookkeeping: sort keys and payloads (empty
    without ``need_backward``), bag counts, the offsets scan and the count of
    ids outside their table."""

    _check_features(weights, ids, lengths, table, pooling, exclude, padding_idx)
    order = _order(weights, table)
    if order is not None:
        ids, lengths, table, pooling, exclude, padding_idx = (
            [x[f] for f in order] for x in (ids, lengths, table, pooling, exclude, padding_idx))
    plan = _plan(weights, table, pooling, exclude, padding_idx)
    res = ops.grouped_forward(plan, ids, lengths, with_backward=need_backward, with_bag_count=True)
    device = weights[0].device
    empty_i32 = torch.empty(0, dtype=torch.int32, device=device)
    keys = res.keys if need_backward else empty_i32
    payload = res.payload if need_backward else empty_i32.clone()
    bag_count = res.bag_count if res.bag_count is not None else torch.empty(0, dtype=torch.float32, device=device)
    offsets = res.offsets if res.offsets is not None else torch.empty(0, dtype=torch.int64, device=device)
    outputs = list(res.outputs)
    if order is not None:
        back = [None] * len(order)
        for i, f in enumerate(order):
            back[f] = outputs[i]
        outputs = back
    return outputs, keys, payload, bag_count, offsets, res.error_count


def _pool_cpu(emb: Tensor, live: Tensor, lengths: Tensor, mean: bool) -> tuple[Tensor, Tensor]:
    """fp32 sums (and weight counts) of flat bags; the reference's index_add_
    pooling (src/model.py:552-570) with fp32 accumulation and one rounding."""

    batch = int(lengths.numel())
    seg = torch.repeat_interleave(torch.arange(batch, dtype=torch.long), lengths.long())
    sums = torch.zeros((batch, emb.size(-1)), dtype=torch.float32)
    counts = torch.zeros(batch, dtype=torch.float32)
    if seg.numel():
        sums.index_add_(0, seg, emb.float() * live.unsqueeze(-1))
        counts.index_add_(0, seg, live)
    if mean:
        sums = sums / counts.clamp(min=1).unsqueeze(-1)
    return sums, counts


@grouped_lookup.register_kernel("cpu")
def _grouped_lookup_cpu(weights, ids, lengths, table, pooling, exclude, padding_idx, need_backward):
    _check_features(weights, ids, lengths, table, pooling, exclude, padding_idx)
    n_ids, rows_out, n_len, pooled_any = _layout(ids, lengths, pooling)
    outputs = []
    bag_count = torch.zeros(max(sum(rows_out), 1) if pooled_any else 0, dtype=torch.float32)
    bad = 0
    base = 0
    for f, x in enumerate(ids):
        w = weights[table[f]]
        flat = x.reshape(-1)
        valid = (flat >= 0) & (flat < w.size(0))
        bad += int((~valid).sum())
        emb = w.index_select(0, torch.where(valid, flat, 0))
        if pooling[f] == 0:
            out = torch.where(valid.unsqueeze(-1), emb, torch.zeros((), dtype=w.dtype))
            outputs.append(out.reshape(*x.shape, w.size(1)))
        else:
            ln = lengths[f]
            if int(ln.sum()) != flat.numel() or bool((ln < 0).any()):
                raise ValueError(
                    f"categorical bag flat length {flat.numel()} != sum(lengths) {int(ln.clamp(min=0).sum())}"
                )
            live = valid & (flat.ne(0) if exclude[f] else torch.ones_like(valid))
            sums, counts = _pool_cpu(emb, live.float(), ln, pooling[f] == 2)
            outputs.append(sums.to(w.dtype))
            bag_count[base: base + counts.numel()] = counts
        base += rows_out[f]
    if pooled_any:
        parts = [lengths[f].to(torch.int64) if pooling[f] != 0 else torch.tensor([n_ids[f]]) for f in range(len(ids))]
        offsets = _offsets_cpu(torch.cat(parts))
    else:
        offsets = torch.empty(0, dtype=torch.int64)
    empty = torch.empty(0, dtype=torch.int32)
    return outputs, empty, empty.clone(), bag_count, offsets, torch.tensor([bad], dtype=torch.int32)


@grouped_lookup.register_fake
def _grouped_lookup_fake(weights, ids, lengths, table, pooling, exclude, padding_idx, need_backward):
    n_ids, rows_out, n_len, pooled_any = _layout(ids, lengths, pooling)
    outputs = []
    for f, x in enumerate(ids):
        w = weights[table[f]]
        shape = (*x.shape, w.size(1)) if pooling[f] == 0 else (lengths[f].size(0), w.size(1))
        outputs.append(w.new_empty(shape))
    w0 = weights[0]
    n = sum(n_ids)
    nk = max(n, 1) if (need_backward and _is_rocm(w0)) else 0
    keys = w0.new_empty(nk, dtype=torch.int32)
    bag_count = w0.new_empty(max(sum(rows_out), 1) if pooled_any else 0, dtype=torch.float32)
    offsets = w0.new_empty(n_len + 1 if pooled_any else 0, dtype=torch.int64)
    return outputs, keys, w0.new_empty(nk, dtype=torch.int32), bag_count, offsets, w0.new_empty(1, dtype=torch.int32)


def _capacities(weights, ids, table) -> list[int]:
    cap = [0] * len(weights)
    for f, x in enumerate(ids):
        cap[table[f]] += int(x.numel())
    return cap


@torch.library.custom_op("mdl_hip::grouped_lookup_backward", mutates_args=(), device_types=_CUDA)
def grouped_lookup_backward(
    weights: list[Tensor], ids: list[Tensor], lengths: list[Optional[Tensor]], table: list[int],
    pooling: list[int], exclude: list[int], padding_idx: list[int], grads: list[Tensor], keys: Tensor,
    payload: Tensor, bag_count: Tensor, offsets: Tensor,
) -> tuple[Tensor, Tensor, Tensor]:
    """Capacity-sized coalesced gradients of every table in two flat buffers
    -- rows int64 and value bytes, laid out by ``ops.coalesced_layout`` (cut
    per table with ``ops.split_coalesced``) -- and their device row counts
    (int64 ``[T]``).  The sort works on copies of the keys and payloads, so the
    op leaves its inputs as they are."""

    order = _order(weights, table)
    if order is not None:
        ids, lengths, table, pooling, exclude, padding_idx, grads = (
            [x[f] for f in order] for x in (ids, lengths, table, pooling, exclude, padding_idx, grads))
    plan = _plan(weights, table, pooling, exclude, padding_idx)
    keys = keys.clone()
    payload = payload.clone()
    n_ids = [int(x.numel()) for x in ids]
    bags = [int(lengths[f].numel()) if pooling[f] != 0 else 0 for f in range(len(ids))]
    feats = ops.build_features(plan, n_ids, bags, [g.data_ptr() for g in grads],
                               [int(g.stride(0)) if g.ndim == 2 else int(g.size(-1)) for g in grads])
    res = ops.ForwardResult(
        plan=plan, device=weights[0].device, ids=ids[0], offsets=offsets if offsets.numel() else None,
        outputs=list(grads), feats=feats, keys=keys, payload=payload,
        bag_count=bag_count if bag_count.numel() else None, error_count=torch.empty(0), count=sum(n_ids),
    )
    rows_all, vbuf, counts, _ = ops.backward_coalesce_padded(res, grads)
    return rows_all, vbuf, counts


def _per_id_grads_cpu(w: Tensor, x: Tensor, ln: Optional[Tensor], g: Tensor, pooling: int, exclude: int,
                      padding_idx: int) -> tuple[Tensor, Tensor]:
    flat = x.reshape(-1)
    valid = (flat >= 0) & (flat < w.size(0))
    dim = int(w.size(1))
    g = g.reshape(-1, dim).float()
    if pooling == 0:
        keep = valid & flat.ne(padding_idx)
        return flat[keep], g[keep]
    live = valid & (flat.ne(0) if exclude else torch.ones_like(valid))
    batch = int(ln.numel())
    seg = torch.repeat_interleave(torch.arange(batch, dtype=torch.long), ln.long())
    counts = torch.zeros(batch, dtype=torch.float32)
    if seg.numel():
        counts.index_add_(0, seg, live.float())
    per_id = g[seg]
    if pooling == 2:
        # the autograd of sums / counts.clamp(min=1) (src/model.py:570): a division
        per_id = per_id / counts.clamp(min=1)[seg].unsqueeze(-1)
    keep = live & flat.ne(padding_idx)
    return flat[keep], per_id[keep]


def _coalesce_padded_cpu(rows: Tensor, vals: Tensor, cap: int, dtype: torch.dtype, dim: int):
    """Sorted unique rows and fp32 segment sums (rounded once to ``dtype``),
    padded to ``cap`` entries like the device path."""

    if rows.numel():
        uniq, inv = torch.unique(rows, sorted=True, return_inverse=True)
        sums = torch.zeros((uniq.numel(), dim), dtype=torch.float32).index_add_(0, inv, vals)
    else:
        uniq = rows.new_empty(0)
        sums = torch.zeros((0, dim), dtype=torch.float32)
    u = int(uniq.numel())
    out_rows = torch.full((cap,), int(uniq[-1]) if u else 0, dtype=torch.int64)
    out_rows[:u] = uniq
    out_vals = torch.zeros((cap, dim), dtype=dtype)
    out_vals[:u] = sums.to(dtype)
    return out_rows, out_vals, u


@grouped_lookup_backward.register_kernel("cpu")
def _grouped_backward_cpu(weights, ids, lengths, table, pooling, exclude, padding_idx, grads, keys, payload,
                          bag_count, offsets):
    cap = _capacities(weights, ids, table)
    layout = ops.coalesced_layout(weights, cap)
    rows_all = torch.empty(max(int(layout["rows_off"][-1]), 1), dtype=torch.int64)
    vbuf = torch.zeros(max(int(layout["val_off"][-1]), 1), dtype=torch.uint8)
    rows, values = ops.split_coalesced(weights, rows_all, vbuf, layout)
    parts = [([], []) for _ in weights]
    for f, x in enumerate(ids):
        t = table[f]
        r, v = _per_id_grads_cpu(weights[t], x, lengths[f], grads[f], pooling[f], exclude[f], padding_idx[f])
        parts[t][0].append(r)
        parts[t][1].append(v)
    counts = []
    for t, w in enumerate(weights):
        r = torch.cat(parts[t][0]) if parts[t][0] else torch.empty(0, dtype=torch.int64)
        v = torch.cat(parts[t][1]) if parts[t][1] else torch.empty((0, int(w.size(1))))
        orow, oval, u = _coalesce_padded_cpu(r, v, cap[t], w.dtype, int(w.size(1)))
        rows[t].copy_(orow)
        values[t].copy_(oval)
        counts.append(u)
    return rows_all, vbuf, torch.tensor(counts, dtype=torch.int64)


@grouped_lookup_backward.register_fake
def _grouped_backward_fake(weights, ids, lengths, table, pooling, exclude, padding_idx, grads, keys, payload,
                           bag_count, offsets):
    layout = ops.coalesced_layout(weights, _capacities(weights, ids, table))
    w0 = weights[0]
    return (w0.new_empty(max(int(layout["rows_off"][-1]), 1), dtype=torch.int64),
            w0.new_empty(max(int(layout["val_off"][-1]), 1), dtype=torch.uint8),
            w0.new_empty(len(weights), dtype=torch.int64))


def _lookup_setup(ctx, inputs, output):
    weights, ids, lengths, table, pooling, exclude, padding_idx, need_backward = inputs
    _, keys, payload, bag_count, offsets, _ = output
    ctx.save_for_backward(*weights, *ids, keys, payload, bag_count, offsets)
    ctx.nw = len(weights)
    ctx.nf = len(ids)
    ctx.lengths = list(lengths)
    ctx.spec = (list(table), list(pooling), list(exclude), list(padding_idx))


def _lookup_backward(ctx, grad_outputs, *_unused):
    saved = ctx.saved_tensors
    weights = list(saved[: ctx.nw])
    ids = list(saved[ctx.nw: ctx.nw + ctx.nf])
    keys, payload, bag_count, offsets = saved[ctx.nw + ctx.nf:]
    table, pooling, exclude, padding_idx = ctx.spec
    grads = []
    for f, g in enumerate(grad_outputs):
        w = weights[table[f]]
        if g is None:
            rows_f = int(ctx.lengths[f].numel()) if pooling[f] != 0 else int(ids[f].numel())
            g = torch.zeros((rows_f, int(w.size(1))), dtype=w.dtype, device=w.device)
        # Row-strided gradients (column slices of one [B, sum(D)] gradient, as
        # a concatenation of the outputs hands back) are read in place.
        grads.append(g if g.ndim == 2 and g.stride(-1) == 1 else g.contiguous())
    rows_all, vbuf, counts = torch.ops.mdl_hip.grouped_lookup_backward(
        weights, ids, ctx.lengths, table, pooling, exclude, padding_idx, grads, keys, payload, bag_count, offsets,
    )
    rows, values = ops.split_coalesced(weights, rows_all, vbuf,
                                       ops.coalesced_layout(weights, _capacities(weights, ids, table)))
    _drop_dead_records()
    wgrads = []
    for t, w in enumerate(weights):
        g = torch.sparse_coo_tensor(rows[t].unsqueeze(0), values[t], tuple(w.shape), is_coalesced=False)
        _note_capacity_grad(w, rows[t], values[t], counts[t: t + 1])
        wgrads.append(g)
    # Same structure as the inputs: a list of tensors gets a list back; a
    # list holding a None (unpooled features' lengths) is one leaf.
    lengths_grad = [None] * ctx.nf if all(ln is not None for ln in ctx.lengths) else None
    return wgrads, [None] * ctx.nf, lengths_grad, None, None, None, None, None


torch.library.register_autograd("mdl_hip::grouped_lookup", _lookup_backward, setup_context=_lookup_setup)


# ------------------------------------------------------------- sequences --


@torch.library.custom_op("mdl_hip::sequence_lookup", mutates_args=(), device_types=_CUDA)
def sequence_lookup(weight: Tensor, ids: Tensor, lengths: Tensor, out_len: int, newest_first: bool,
                    padding_idx: int, need_backward: bool) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Right-aligned window ``[B, out_len, dim]``, its mask, the backward's
    sort keys/payloads (empty without ``need_backward``) and the count of ids
    outside the table."""

    res = ops.sequence_lookup(weight, ids, lengths, out_len=out_len,
                              order="newest_to_oldest" if newest_first else "oldest_to_newest",
                              padding_idx=padding_idx, with_backward=need_backward)
    empty = torch.empty(0, dtype=torch.int32, device=weight.device)
    keys = res.keys if need_backward else empty
    payload = res.payload if need_backward else empty.clone()
    return res.outputs[0], res.keep[0], keys, payload, res.error_count


def _window_cpu(ids: Tensor, lengths: Tensor, out_len: int, newest_first: bool):
    """(mask [B, out_len], source position [B, out_len]) of the window: the
    reference's clamp of the lengths to the output width and of the source
    position to the input width (src/model.py:2998-3016), so a length past
    the input repeats its last element; an empty input masks everything."""

    batch, in_len = ids.shape
    n = lengths.to(torch.int64).clamp(min=0).clamp(max=out_len)
    if in_len == 0:
        n = torch.zeros_like(n)
    start = out_len - n
    p = torch.arange(out_len).unsqueeze(0)
    mask = p >= start.unsqueeze(1)
    rel = p - start.unsqueeze(1)
    src = (n.unsqueeze(1) - 1 - rel) if newest_first else rel
    src = src.clamp(max=max(in_len - 1, 0))
    return mask, torch.where(mask, src, 0)


@sequence_lookup.register_kernel("cpu")
def _sequence_lookup_cpu(weight, ids, lengths, out_len, newest_first, padding_idx, need_backward):
    mask, src = _window_cpu(ids, lengths, out_len, newest_first)
    rows = torch.gather(ids, 1, src) if ids.size(1) else torch.zeros_like(src)
    valid = (rows >= 0) & (rows < weight.size(0))
    bad = int((mask & ~valid).sum())
    live = mask & valid
    out = weight.index_select(0, torch.where(live, rows, 0).reshape(-1)).reshape(*rows.shape, weight.size(1))
    out = torch.where(live.unsqueeze(-1), out, torch.zeros((), dtype=weight.dtype))
    empty = torch.empty(0, dtype=torch.int32)
    return out, mask, empty, empty.clone(), torch.tensor([bad], dtype=torch.int32)


@sequence_lookup.register_fake
def _sequence_lookup_fake(weight, ids, lengths, out_len, newest_first, padding_idx, need_backward):
    batch = ids.size(0)
    nk = max(int(batch * out_len), 1) if (need_backward and _is_rocm(weight)) else 0
    return (weight.new_empty((batch, out_len, weight.size(1))), ids.new_empty((batch, out_len), dtype=torch.bool),
            ids.new_empty(nk, dtype=torch.int32), ids.new_empty(nk, dtype=torch.int32),
            ids.new_empty(1, dtype=torch.int32))


@torch.library.custom_op("mdl_hip::sequence_lookup_backward", mutates_args=(), device_types=_CUDA)
def sequence_lookup_backward(weight: Tensor, ids: Tensor, lengths: Tensor, out_len: int, newest_first: bool,
                             padding_idx: int, grad: Tensor, keys: Tensor, payload: Tensor
                             ) -> tuple[Tensor, Tensor, Tensor]:
    """Capacity-sized coalesced gradient of the window gather (capacity: the
    window positions, ``batch * out_len``) and its device row count (int64
    [1]).  The sort works on copies of the keys and payloads."""

    n = int(ids.size(0)) * int(out_len)
    if keys.numel() < n or payload.numel() < n:
        raise ValueError("sequence sort keys hold one entry per window position (batch * out_len)")
    keys = keys.clone()
    payload = payload.clone()
    plan = ops.GroupPlan()
    plan.add_feature(weight, pooling="none", padding_idx=padding_idx)
    feats = ops.sequence_feature(weight, padding_idx=padding_idx)
    feats["num_ids"] = n
    res = ops.ForwardResult(
        plan=plan, device=weight.device, ids=ids, offsets=None, outputs=[grad], feats=feats, keys=keys,
        payload=payload, bag_count=None, error_count=torch.empty(0), count=n,
    )
    rows_all, vbuf, counts, layout = ops.backward_coalesce_padded(res, [grad.reshape(-1, int(weight.size(1)))])
    rows, values = ops.split_coalesced([weight], rows_all, vbuf, layout)
    # views of two different buffers that are not returned: no output aliases another
    return rows[0], values[0], counts


@sequence_lookup_backward.register_kernel("cpu")
def _sequence_backward_cpu(weight, ids, lengths, out_len, newest_first, padding_idx, grad, keys, payload):
    mask, src = _window_cpu(ids, lengths, out_len, newest_first)
    rows = torch.gather(ids, 1, src) if ids.size(1) else torch.zeros_like(src)
    keep = mask & (rows >= 0) & (rows < weight.size(0)) & rows.ne(padding_idx)
    dim = int(weight.size(1))
    r, v, u = _coalesce_padded_cpu(rows[keep], grad.float()[keep].reshape(-1, dim), int(ids.size(0)) * int(out_len),
                                   weight.dtype, dim)
    return r, v, torch.tensor([u], dtype=torch.int64)


@sequence_lookup_backward.register_fake
def _sequence_backward_fake(weight, ids, lengths, out_len, newest_first, padding_idx, grad, keys, payload):
    n = int(ids.size(0)) * int(out_len)
    return (weight.new_empty(n, dtype=torch.int64), weight.new_empty((n, weight.size(1))),
            weight.new_empty(1, dtype=torch.int64))


def _sequence_setup(ctx, inputs, output):
    weight, ids, lengths, out_len, newest_first, padding_idx, need_backward = inputs
    _, mask, keys, payload, _ = output
    ctx.save_for_backward(weight, ids, lengths, keys, payload)
    ctx.args = (int(out_len), bool(newest_first), int(padding_idx))
    ctx.mark_non_differentiable(mask)


def _sequence_backward(ctx, grad_out, *_unused):
    weight, ids, lengths, keys, payload = ctx.saved_tensors
    out_len, newest_first, padding_idx = ctx.args
    if grad_out is None:
        grad_out = torch.zeros((ids.size(0), out_len, weight.size(1)), dtype=weight.dtype, device=weight.device)
    rows, values, count = torch.ops.mdl_hip.sequence_lookup_backward(
        weight, ids, lengths, out_len, newest_first, padding_idx, grad_out.contiguous(), keys, payload,
    )
    _note_capacity_grad(weight, rows, values, count)
    g = torch.sparse_coo_tensor(rows.unsqueeze(0), values, tuple(weight.shape), is_coalesced=False)
    return g, None, None, None, None, None, None


torch.library.register_autograd("mdl_hip::sequence_lookup", _sequence_backward, setup_context=_sequence_setup)


# ----------------------------------------------------------- coalescing --


@torch.library.custom_op("mdl_hip::sparse_coalesce", mutates_args=(), device_types=_CUDA)
def sparse_coalesce(indices: Tensor, values: Tensor, num_rows: int) -> tuple[Tensor, Tensor]:
    """Rows ascending and unique with their summed values (one host read to
    size them, like Tensor.coalesce())."""

    return ops.coalesce_rows(indices, values, num_rows)


@sparse_coalesce.register_kernel("cpu")
def _sparse_coalesce_cpu(indices, values, num_rows):
    g = torch.sparse_coo_tensor(indices.reshape(1, -1), values, (num_rows, values.size(1))).coalesce()
    return g.indices()[0].clone(), g.values().clone()


@sparse_coalesce.register_fake
def _sparse_coalesce_fake(indices, values, num_rows):
    ctx = torch.library.get_ctx()
    u = ctx.new_dynamic_size()
    return indices.new_empty(u), values.new_empty((u, values.size(1)))


@torch.library.custom_op("mdl_hip::sparse_coalesce_padded", mutates_args=(), device_types=_CUDA)
def sparse_coalesce_padded(indices: Tensor, values: Tensor, num_rows: int) -> tuple[Tensor, Tensor, Tensor]:
    """Capacity-sized coalesce (no host read): ``(rows [n], values [n, dim],
    count)``, the first ``count`` rows ascending and unique, the rest
    repeating the last row with zero values."""

    return ops.coalesce_rows_padded(indices, values, num_rows)


@sparse_coalesce_padded.register_kernel("cpu")
def _sparse_coalesce_padded_cpu(indices, values, num_rows):
    keep = (indices >= 0) & (indices < num_rows)
    dim = int(values.size(1))
    r, v, u = _coalesce_padded_cpu(indices[keep], values.float()[keep], int(indices.numel()), values.dtype, dim)
    return r, v, torch.tensor([u], dtype=torch.int64)


@sparse_coalesce_padded.register_fake
def _sparse_coalesce_padded_fake(indices, values, num_rows):
    n = int(indices.numel())
    return indices.new_empty(n, dtype=torch.int64), values.new_empty((n, values.size(1))), \
        indices.new_empty(1, dtype=torch.int64)


# --------------------------------------------------------------- update --


@torch.library.custom_op("mdl_hip::rowwise_adagrad_", mutates_args=("weight", "accumulator"), device_types=_CUDA)
def rowwise_adagrad_(weight: Tensor, accumulator: Tensor, rows: Tensor, values: Tensor, lr: float,
                     eps: float) -> None:
    ops.rowwise_adagrad_(weight, accumulator, rows, values, lr=lr, eps=eps)


@rowwise_adagrad_.register_kernel("cpu")
def _rowwise_adagrad_cpu(weight, accumulator, rows, values, lr, eps):
    """The CPU branch of ShardedRowWiseAdagrad.step (src/optim.py:359-376):
    the update is rounded to the weight dtype, then added."""

    if rows.numel() == 0:
        return
    state_values = values if values.dtype == torch.float32 else values.float()
    accumulator.index_add_(0, rows, state_values.square().mean(dim=1))
    den = accumulator.index_select(0, rows).sqrt_().add_(eps).unsqueeze(1)
    update = state_values / den
    if update.dtype != weight.dtype:
        update = update.to(dtype=weight.dtype)
    weight.index_add_(0, rows, update, alpha=-lr)


@rowwise_adagrad_.register_fake
def _rowwise_adagrad_fake(weight, accumulator, rows, values, lr, eps):
    return None


@torch.library.custom_op("mdl_hip::grouped_rowwise_adagrad_", mutates_args=("weights", "accumulators"),
                         device_types=_CUDA)
def grouped_rowwise_adagrad_(weights: list[Tensor], accumulators: list[Tensor], rows: list[Tensor],
                             values: list[Tensor], counts: list[Optional[Tensor]], lrs: list[float],
                             eps: float) -> None:
    """Row-wise Adagrad of every table in one launch; table i updates
    ``rows[i][:counts[i]]`` (the count read on the device; None: all)."""

    ops.grouped_rowwise_adagrad_(weights, accumulators, rows, values, counts, lrs, eps=eps)


@grouped_rowwise_adagrad_.register_kernel("cpu")
def _grouped_adagrad_cpu(weights, accumulators, rows, values, counts, lrs, eps):
    for w, a, r, v, c, lr in zip(weights, accumulators, rows, values, counts, lrs):
        n = int(r.numel()) if c is None else int(c.reshape(-1)[0])
        _rowwise_adagrad_cpu(w, a, r[:n], v[:n], lr, eps)


@grouped_rowwise_adagrad_.register_fake
def _grouped_adagrad_fake(weights, accumulators, rows, values, counts, lrs, eps):
    return None


# ------------------------------------------- gradients the optimizer knows --

# Capacity-sized gradients this module emitted, by parameter: the optimizer
# finds their device row count here instead of coalescing them again.
# Autograd's AccumulateGrad may re-wrap a sparse gradient around the same
# index and value storage; the record is matched by storage.  A gradient
# accumulated over several backward passes has new storage and is coalesced
# normally.
_CAPACITY_GRADS: dict[int, tuple] = {}


def _note_capacity_grad(parameter: Tensor, rows: Tensor, values: Tensor, count: Tensor) -> None:
    _CAPACITY_GRADS[id(parameter)] = (weakref.ref(parameter), rows, values, count)


def _drop_dead_records() -> None:
    """Forget records of parameters that no longer exist (once per backward)."""

    for key in [k for k, rec in _CAPACITY_GRADS.items() if rec[0]() is None]:
        del _CAPACITY_GRADS[key]


def capacity_grad(parameter: Tensor, grad: Tensor) -> Optional[tuple[Tensor, Tensor, Tensor]]:
    """``(rows, values, count)`` when ``grad`` is the capacity-sized gradient
    last emitted for ``parameter``, else None."""

    entry = _CAPACITY_GRADS.get(id(parameter))
    if entry is None or entry[0]() is not parameter:
        return None
    _, rows, values, count = entry
    idx, val = grad._indices(), grad._values()
    if (idx.data_ptr() == rows.data_ptr() and val.data_ptr() == values.data_ptr()
            and idx.size(-1) == rows.numel() and tuple(val.shape) == tuple(values.shape)):
        return rows, values, count
    return None


def forget_capacity_grad(parameter: Tensor) -> None:
    _CAPACITY_GRADS.pop(id(parameter), None)
