"""The sparse path as torch.library operators, namespace ``mdl_hip``.

The schemas and their ROCm kernels live in the C++ extension
``libmdl_torch.so`` (mdl_amd/csrc/torch_ops.cpp), which calls the
hand-written gfx950 kernels of libmdl_hip.so through its C ABI on the current
HIP stream; importing this module loads it and raises when it is missing.
This module registers on those schemas:

* CPU kernels: PyTorch CPU operations with the reference's CPU semantics, so
  modules whose parameters live on the CPU work as in the reference
  (src/embeddings.py:468-473, src/model.py:509-678, src/optim.py:359-376);
* fake kernels: shapes only, for tracing and ``torch.compile``;
* the autograd formulas of the two lookups.

Public ops:

``mdl_hip::bucketize``                 pre_hashed / mod bucketing (src/features.py:360-376, src/benchmark.py:1246-1250)
``mdl_hip::bag_truncate``              list features to CSR bags (src/dataloader.py:8565-8665)
``mdl_hip::lengths_to_offsets``        CSR offsets of bag lengths
``mdl_hip::grouped_lookup``            grouped lookup + sum/mean bag pooling (src/embeddings.py:1646-1709, src/model.py:509-678)
``mdl_hip::grouped_lookup_backward``   its coalesced sparse weight gradients, capacity-sized (no host read)
``mdl_hip::sequence_lookup``           right-aligned sequence window gather (src/model.py:2989-3100)
``mdl_hip::sequence_lookup_backward``  its coalesced sparse weight gradient, capacity-sized
``mdl_hip::sparse_coalesce``           sort + unique + segment sum of a COO gradient (src/optim.py:321-324)
``mdl_hip::sparse_coalesce_padded``    the same, capacity-sized (no host read)
``mdl_hip::rowwise_adagrad_``          row-wise Adagrad of one table (src/optim.py:68-108, CPU :359-376)
``mdl_hip::grouped_rowwise_adagrad_``  row-wise Adagrad of many tables in one launch, row counts read on device

The C++ extension also defines the whole-step helpers the modules call
(``grouped_lookup_weight_grads``, ``rowwise_adagrad_step_``, ...) and the
fused step's launches (``packed_forward_``, ``fused_backward_rowwise_adagrad_``,
...).

Sparse gradients of the lookups come in one of two modes
(:func:`set_sparse_grad_mode`):

* ``"coalesced"`` (default): each table's gradient is coalesced -- rows
  ascending and unique, ``is_coalesced()`` true -- so the trainer's
  ``grad.coalesce()`` (src/train.py:5738, src/optim.py:323-324) returns it as
  it is.  Sizing them costs one batched device-to-host read of every table's
  row count per backward.
* ``"capacity"``: table t's gradient has ``cap_t`` entries (its id count, a
  bound on its distinct rows that the host knows from the shapes); the first
  U_t are the coalesced rows and the rest repeat the last row with zero
  values.  The pair is a valid uncoalesced COO gradient with the coalesced
  sum and needs no host read; ``ShardedRowWiseAdagrad`` and ``mdl_amd.clip``
  read U_t on the device.  A trainer that keeps the reference's
  ``grad.coalesce()`` would coalesce such gradients again through ATen.
"""

from __future__ import annotations

import os
from pathlib import Path
from typing import Optional

import torch
from torch import Tensor

from . import _lib, ops

TORCH_LIB_PATH = Path(__file__).resolve().parent / "libmdl_torch.so"

_POOL = {0: "none", 1: "sum", 2: "mean"}
_CUDA = "cuda"


def _load() -> None:
    _lib.lib()  # the C ABI and its version check
    if not TORCH_LIB_PATH.exists():
        raise RuntimeError(
            f"{TORCH_LIB_PATH.name} not found at {TORCH_LIB_PATH}; build it with `python mdl_amd/build.py` "
            "(the torch.library extension of the mdl_hip operators)"
        )
    torch.ops.load_library(str(TORCH_LIB_PATH))


_load()

_GRAD_MODES = ("coalesced", "capacity")
_grad_mode = os.environ.get("MDL_SPARSE_GRADS", "coalesced")
if _grad_mode not in _GRAD_MODES:
    raise ValueError(f"MDL_SPARSE_GRADS must be one of {_GRAD_MODES}, got {_grad_mode!r}")
# the modules' backward in C++ reads the mode from the extension
torch.ops.mdl_hip.set_exact_sparse_grads(_grad_mode == "coalesced")


def set_sparse_grad_mode(mode: str) -> None:
    """``"coalesced"`` (exact coalesced sparse gradients, one device-to-host
    read per backward) or ``"capacity"`` (capacity-sized gradients, no host
    read); see the module docstring."""

    global _grad_mode
    if mode not in _GRAD_MODES:
        raise ValueError(f"sparse gradient mode must be one of {_GRAD_MODES}")
    _grad_mode = mode
    torch.ops.mdl_hip.set_exact_sparse_grads(mode == "coalesced")


def sparse_grad_mode() -> str:
    return _grad_mode


def _is_rocm(t: Tensor) -> bool:
    return t.device.type == _CUDA


def _eager(t: Tensor) -> bool:
    """A plain tensor with data, not a fake or functional one being traced."""

    return type(t) is Tensor or type(t) is torch.nn.Parameter


def _cpu_kernel(name: str):
    """Register the decorated function as the CPU kernel of mdl_hip::name."""

    def deco(fn):
        torch.library.register_kernel(f"mdl_hip::{name}", "cpu", fn)
        return fn

    return deco


def _fake_kernel(name: str):
    """Register the decorated function as the fake kernel of mdl_hip::name."""

    def deco(fn):
        torch.library.register_fake(f"mdl_hip::{name}", fn)
        return fn

    return deco


# ------------------------------------------------------------- bucketing --


@_cpu_kernel("bucketize")
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


@_fake_kernel("bucketize")
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


@_cpu_kernel("bag_truncate")
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


@_fake_kernel("bag_truncate")
def _bag_truncate_fake(values, offsets, valid, row_valid, max_length, truncation, bucket, num_buckets,
                       validate_nonzero):
    rows = offsets.size(0) - 1
    return (values.new_empty(values.size(0), dtype=torch.int64), offsets.new_empty(rows, dtype=torch.int64),
            offsets.new_empty(rows + 1, dtype=torch.int64), values.new_empty(1, dtype=torch.int32))


@_cpu_kernel("lengths_to_offsets")
def _offsets_cpu(lengths):
    out = torch.zeros(lengths.numel() + 1, dtype=torch.int64)
    torch.cumsum(lengths.to(torch.int64), 0, out=out[1:])
    return out


@_fake_kernel("lengths_to_offsets")
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
    """Feature order of a device call (the C++ extension's rule): the
    callers' order (None), except that a call over 2^32 - 1 table rows or more
    looks its features up sorted by table, so that each key group's features
    are consecutive (its keys one stretch)."""

    order = torch.ops.mdl_hip.lookup_order(list(weights), [int(t) for t in table])
    return list(order) if order else None


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


@_cpu_kernel("grouped_lookup")
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


@_fake_kernel("grouped_lookup")
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


@_cpu_kernel("grouped_lookup_backward")
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


@_fake_kernel("grouped_lookup_backward")
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


def lookup_weight_grads(weights, ids, lengths, spec, aux, grad_outputs) -> list[Tensor]:
    """Sparse gradients of every table of a grouped lookup from the upstream
    gradients of its outputs (None: zeros).  ``spec`` is (table, pooling,
    exclude, padding_idx) and ``aux`` the forward's (keys, payload,
    bag_count, offsets)."""

    keys, payload, bag_count, offsets = aux
    table, pooling, exclude, padding_idx = spec
    grads = list(grad_outputs)
    for f, g in enumerate(grads):
        if g is None:
            w = weights[table[f]]
            rows_f = int(lengths[f].numel()) if pooling[f] != 0 else int(ids[f].numel())
            grads[f] = torch.zeros((rows_f, int(w.size(1))), dtype=w.dtype, device=w.device)
    # Row-strided gradients (column slices of one [B, sum(D)] gradient, as a
    # concatenation of the outputs hands back) are read in place.
    if _eager(keys):
        # the sparse gradients of every table from one call
        return list(torch.ops.mdl_hip.grouped_lookup_weight_grads(
            weights, ids, lengths, table, pooling, exclude, padding_idx, grads, keys, payload, bag_count,
            offsets, _grad_mode == "coalesced",
        ))
    # traced (fake or functional tensors): the public op and capacity-sized
    # COO tensors, which need no data
    rows_all, vbuf, counts = torch.ops.mdl_hip.grouped_lookup_backward(
        weights, ids, lengths, table, pooling, exclude, padding_idx, grads, keys, payload, bag_count, offsets,
    )
    rows, values = ops.split_coalesced(weights, rows_all, vbuf,
                                       ops.coalesced_layout(weights, _capacities(weights, ids, table)))
    return [torch.sparse_coo_tensor(r.unsqueeze(0), v, tuple(w.shape), is_coalesced=False)
            for w, r, v in zip(weights, rows, values)]


def _lookup_backward(ctx, grad_outputs, *_unused):
    saved = ctx.saved_tensors
    weights = list(saved[: ctx.nw])
    ids = list(saved[ctx.nw: ctx.nw + ctx.nf])
    wgrads = lookup_weight_grads(weights, ids, ctx.lengths, ctx.spec, saved[ctx.nw + ctx.nf:], grad_outputs)
    # Same structure as the inputs: a list of tensors gets a list back; a
    # list holding a None (unpooled features' lengths) is one leaf.
    lengths_grad = [None] * ctx.nf if all(ln is not None for ln in ctx.lengths) else None
    return wgrads, [None] * ctx.nf, lengths_grad, None, None, None, None, None


torch.library.register_autograd("mdl_hip::grouped_lookup", _lookup_backward, setup_context=_lookup_setup)


# ------------------------------------------------------------- sequences --


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


@_cpu_kernel("sequence_lookup")
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


@_fake_kernel("sequence_lookup")
def _sequence_lookup_fake(weight, ids, lengths, out_len, newest_first, padding_idx, need_backward):
    batch = ids.size(0)
    nk = max(int(batch * out_len), 1) if (need_backward and _is_rocm(weight)) else 0
    return (weight.new_empty((batch, out_len, weight.size(1))), ids.new_empty((batch, out_len), dtype=torch.bool),
            ids.new_empty(nk, dtype=torch.int32), ids.new_empty(nk, dtype=torch.int32),
            ids.new_empty(1, dtype=torch.int32))


@_cpu_kernel("sequence_lookup_backward")
def _sequence_backward_cpu(weight, ids, lengths, out_len, newest_first, padding_idx, grad, keys, payload):
    mask, src = _window_cpu(ids, lengths, out_len, newest_first)
    rows = torch.gather(ids, 1, src) if ids.size(1) else torch.zeros_like(src)
    keep = mask & (rows >= 0) & (rows < weight.size(0)) & rows.ne(padding_idx)
    dim = int(weight.size(1))
    r, v, u = _coalesce_padded_cpu(rows[keep], grad.float()[keep].reshape(-1, dim), int(ids.size(0)) * int(out_len),
                                   weight.dtype, dim)
    return r, v, torch.tensor([u], dtype=torch.int64)


@_fake_kernel("sequence_lookup_backward")
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
    if _eager(rows):
        g = torch.ops.mdl_hip.capacity_sparse_grad(weight, rows, values, count, _grad_mode == "coalesced")
    else:
        g = torch.sparse_coo_tensor(rows.unsqueeze(0), values, tuple(weight.shape), is_coalesced=False)
    return g, None, None, None, None, None, None


torch.library.register_autograd("mdl_hip::sequence_lookup", _sequence_backward, setup_context=_sequence_setup)


# ----------------------------------------------------------- coalescing --


@_cpu_kernel("sparse_coalesce")
def _sparse_coalesce_cpu(indices, values, num_rows):
    g = torch.sparse_coo_tensor(indices.reshape(1, -1), values, (num_rows, values.size(1))).coalesce()
    return g.indices()[0].clone(), g.values().clone()


@_fake_kernel("sparse_coalesce")
def _sparse_coalesce_fake(indices, values, num_rows):
    ctx = torch.library.get_ctx()
    u = ctx.new_dynamic_size()
    return indices.new_empty(u), values.new_empty((u, values.size(1)))


@_cpu_kernel("sparse_coalesce_padded")
def _sparse_coalesce_padded_cpu(indices, values, num_rows):
    keep = (indices >= 0) & (indices < num_rows)
    dim = int(values.size(1))
    r, v, u = _coalesce_padded_cpu(indices[keep], values.float()[keep], int(indices.numel()), values.dtype, dim)
    return r, v, torch.tensor([u], dtype=torch.int64)


@_fake_kernel("sparse_coalesce_padded")
def _sparse_coalesce_padded_fake(indices, values, num_rows):
    n = int(indices.numel())
    return indices.new_empty(n, dtype=torch.int64), values.new_empty((n, values.size(1))), \
        indices.new_empty(1, dtype=torch.int64)


# --------------------------------------------------------------- update --


@_cpu_kernel("rowwise_adagrad_")
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


@_fake_kernel("rowwise_adagrad_")
def _rowwise_adagrad_fake(weight, accumulator, rows, values, lr, eps):
    return None


@_cpu_kernel("grouped_rowwise_adagrad_")
def _grouped_adagrad_cpu(weights, accumulators, rows, values, counts, lrs, eps):
    for w, a, r, v, c, lr in zip(weights, accumulators, rows, values, counts, lrs):
        n = int(r.numel()) if c is None else int(c.reshape(-1)[0])
        _rowwise_adagrad_cpu(w, a, r[:n], v[:n], lr, eps)


@_fake_kernel("grouped_rowwise_adagrad_")
def _grouped_adagrad_fake(weights, accumulators, rows, values, counts, lrs, eps):
    return None


# ------------------------------------------- gradients the optimizer knows --


def capacity_grad(parameter: Tensor, grad: Tensor) -> Optional[tuple[Tensor, Tensor, Tensor]]:
    """``(rows, values, count)`` when ``grad`` is the capacity-sized gradient
    last emitted for ``parameter`` (the extension's record), else None."""

    rec = torch.ops.mdl_hip.capacity_grad_record(parameter, grad)
    return (rec[0], rec[1], rec[2]) if rec else None


def forget_capacity_grad(parameter: Tensor) -> None:
    torch.ops.mdl_hip.forget_capacity_grad(parameter)
