"""CPU oracle of the reference sparse path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may use this module, and only as the checker (or the timed CPU
baseline); the product (``mdl_amd``) never imports it.

The heavy loops are the plain-C restatement in ``oracle/mdl_oracle.c``
(built by ``oracle/Makefile`` into ``oracle/_build/liboracle.so``); the rest
is numpy.  Each function names the reference lines it follows and how it is
pinned (see ``tests/test_oracle.py``):

* bucketize_pre_hashed -- src/features.py:360-376; pinned by the golden
  vectors of tests/test_direct_id.py:183-240 and tests/test_multivalue_features.py:38-93
  (via tests/golden/reference_vectors.json) and by Python's arbitrary-precision
  ``(v & (B-1)) + 1`` on random int64 including INT64_MIN/INT64_MAX.
* bucketize_mod -- src/benchmark.py:1246-1250; pinned by Python's floor-mod
  ``1 + (v - 1) % (N - 1)`` on random int64 including the extremes.
* bag_csr (host, in mdl_amd.features) -- pinned by the same golden vectors.
* bag_truncate -- src/dataloader.py:8565-8640 (Arrow list truncation,
  lengths, flatten); pinned by the same golden vectors in Arrow layout, by
  pyarrow's own ``list_slice`` / ``list_value_length`` / ``list_flatten``
  (library) and by the per-row brute force ``bag_csr`` on random lists.
* pool -- src/model.py:509-570; pinned by the closed-form vectors of
  tests/test_multivalue_features.py:95-120 and by torch's
  ``F.embedding_bag(mode="sum"/"mean")`` and ``_mean_pool``-style index_add_
  formulas on random bags (library routines, CPU).
* pool_rows / pool_rows_padded / pool_rows_backward -- src/model.py:509-587
  on already-embedded rows; pinned by the vectors of
  tests/test_multivalue_features.py:95-121, by torch's ``F.embedding_bag``
  (weighted sum / mean, library, CPU) and its autograd, and by the adjoint
  identity <pool(E), G> = <E, pool_backward(G)> of a linear map.
* sequence_gather -- src/model.py:2989-3100; pinned by a brute-force
  per-position definition and by the reference's padded vectors
  (tests/test_direct_id.py:242-280 layout).
* coalesce -- torch.sparse_coo_tensor(...).coalesce() (library, CPU) and
  torch.unique(sorted, return_inverse, return_counts).
* rowwise_adagrad -- src/optim.py:31-62; pinned by the closed-form cases of
  tests/test_rowwise_adagrad.py:40-128 and tests/test_sharded_embedding.py:647-699.
* clip_grad_norm -- src/train.py:5745-5826; pinned by
  torch.nn.utils.clip_grad_norm_ (same max_norm / (norm + 1e-6) clamped
  coefficient; library, CPU) and by the no-op case norm <= max_norm.
* sparse_step -- composition of the above; pinned by comparing it with the
  separately pinned pieces on random workloads.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

_DIR = Path(__file__).resolve().parent
_SO = _DIR / "_build" / "liboracle.so"
_LIB: ctypes.CDLL | None = None

_P = ctypes.c_void_p


def build() -> Path:
    subprocess.run(["make", "-C", str(_DIR)], check=True, stdout=subprocess.DEVNULL)
    return _SO


def _lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not _SO.exists():
            build()
        lib = ctypes.CDLL(str(_SO))
        lib.oracle_bucketize_pre_hashed.restype = ctypes.c_int64
        lib.oracle_bucketize_pre_hashed.argtypes = [_P, _P, ctypes.c_int64, ctypes.c_int64, _P]
        lib.oracle_bucketize_mod.restype = None
        lib.oracle_bucketize_mod.argtypes = [_P, _P, ctypes.c_int64, ctypes.c_int64, _P]
        lib.oracle_pool.restype = None
        lib.oracle_pool.argtypes = [_P, ctypes.c_int64, ctypes.c_int32, _P, _P, ctypes.c_int64,
                                    ctypes.c_int32, ctypes.c_int32, _P, _P]
        lib.oracle_coalesce.restype = ctypes.c_int64
        lib.oracle_coalesce.argtypes = [_P, _P, ctypes.c_int64, ctypes.c_int32, _P, _P]
        lib.oracle_rowwise_adagrad.restype = None
        lib.oracle_rowwise_adagrad.argtypes = [_P, ctypes.c_int32, ctypes.c_int64, ctypes.c_int32, _P, _P,
                                               ctypes.c_int64, _P, ctypes.c_double, ctypes.c_double]
        lib.oracle_sparse_step.restype = None
        lib.oracle_sparse_step.argtypes = [ctypes.c_int32] + [_P] * 9 + [ctypes.c_int64, _P, _P,
                                           ctypes.c_int32, _P, _P, _P, _P, _P, ctypes.c_double,
                                           ctypes.c_double]
        _LIB = lib
    return _LIB


def _c(a: np.ndarray, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


# ------------------------------------------------------------- bf16 --


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (NaN stays NaN)."""

    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    r = np.where(nan, (u >> 16) | 0x40, r)
    return r.astype(np.uint16)


def round_bf16(x: np.ndarray) -> np.ndarray:
    return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(x, dtype=np.float32)))


# --------------------------------------------------------------- bucketing --


def bucketize_pre_hashed(raw: np.ndarray, num_buckets: int, valid: np.ndarray | None = None):
    """``((uint64)raw & (B-1)) + 1``, null -> 0; returns (ids, non-null zero count)."""

    raw = _c(raw, np.int64)
    out = np.empty_like(raw)
    v = None if valid is None else _c(valid, np.uint8)
    zeros = _lib().oracle_bucketize_pre_hashed(_p(raw), _p(v), raw.size, int(num_buckets), _p(out))
    return out, int(zeros)


def bucketize_mod(raw: np.ndarray, num_embeddings: int, valid: np.ndarray | None = None) -> np.ndarray:
    raw = _c(raw, np.int64)
    out = np.empty_like(raw)
    v = None if valid is None else _c(valid, np.uint8)
    _lib().oracle_bucketize_mod(_p(raw), _p(v), raw.size, int(num_embeddings), _p(out))
    return out


# ----------------------------------------------------------------- forward --


def bag_truncate(offsets: np.ndarray, values: np.ndarray, valid: np.ndarray | None, row_valid: np.ndarray | None,
                 max_length: int | None, truncation: str):
    """List array -> (kept raw values, their validity, per-row kept lengths):
    the reference's truncation of Arrow lists (src/dataloader.py:8565-8604,
    head = ``list_slice(0, max_length)``, tail = the last ``max_length``
    elements by rebuilt offsets) then ``list_value_length`` with nulls as 0
    and ``list_flatten`` (:8634-8640).  The tail rebuild reads the raw
    offsets of every row and makes a list array without a validity bitmap,
    so a null row keeps the last elements of its span there.  Offsets are
    assumed well formed."""

    offsets = np.asarray(offsets, dtype=np.int64)
    lengths = offsets[1:] - offsets[:-1]
    if row_valid is not None and not (truncation == "tail" and max_length is not None):
        lengths = np.where(np.asarray(row_valid) != 0, lengths, 0)
    take = lengths if max_length is None else np.minimum(lengths, int(max_length))
    starts = offsets[:-1] if truncation == "head" else offsets[1:] - take
    total = int(take.sum())
    row_ids = np.repeat(np.arange(take.size, dtype=np.int64), take)
    within = np.arange(total, dtype=np.int64) - np.repeat(np.cumsum(take) - take, take)
    src = starts[row_ids] + within
    vals = np.asarray(values, dtype=np.int64)[src]
    ok = np.ones(total, dtype=np.uint8) if valid is None else (np.asarray(valid)[src] != 0).astype(np.uint8)
    return vals, ok, take.astype(np.int64)


def offsets_of(lengths: np.ndarray) -> np.ndarray:
    lengths = np.asarray(lengths, dtype=np.int64)
    out = np.zeros(lengths.size + 1, dtype=np.int64)
    np.cumsum(lengths, out=out[1:])
    return out


def gather(weight: np.ndarray, ids: np.ndarray) -> np.ndarray:
    """F.embedding forward (src/embeddings.py:468-473): rows in fp64."""

    return np.asarray(weight, dtype=np.float64)[np.asarray(ids, dtype=np.int64)]


def pool(weight: np.ndarray, ids: np.ndarray, lengths: np.ndarray, mode: str, null_policy: str):
    """Bag pooling; returns (out fp64 [B, dim], counts fp64 [B])."""

    w = _c(weight, np.float32)
    ids = _c(ids, np.int64)
    offs = offsets_of(lengths)
    nb = offs.size - 1
    dim = w.shape[1]
    out = np.empty((nb, dim), dtype=np.float64)
    cnt = np.empty(nb, dtype=np.float64)
    code = {"sum": 1, "mean": 2}[mode]
    _lib().oracle_pool(_p(w), w.shape[0], dim, _p(ids), _p(offs), nb, code,
                       1 if null_policy == "exclude" else 0, _p(out), _p(cnt))
    return out, cnt


def pool_rows(embedded: np.ndarray, indices: np.ndarray, lengths: np.ndarray, mode: str,
              null_policy: str):
    """_mean_pool_categorical_bag on already-embedded rows, flat layout
    (src/model.py:552-570): w_i = (id_i != 0) under "exclude" else 1,
    sums[b] = sum_i w_i e_i, counts[b] = sum_i w_i, mean = sums / max(counts, 1).
    Returns (out fp64 [B, dim], counts fp64 [B])."""

    e = np.asarray(embedded, dtype=np.float64)
    ids = np.asarray(indices, dtype=np.int64)
    offs = offsets_of(lengths)
    B = offs.size - 1
    seg = np.repeat(np.arange(B), np.diff(offs))
    w = (ids != 0).astype(np.float64) if null_policy == "exclude" else np.ones(ids.size)
    sums = np.zeros((B, e.shape[1]))
    cnt = np.zeros(B)
    np.add.at(sums, seg, e * w[:, None])
    np.add.at(cnt, seg, w)
    if mode == "mean":
        sums /= np.maximum(cnt, 1.0)[:, None]
    return sums, cnt


def pool_rows_padded(embedded: np.ndarray, indices: np.ndarray, lengths: np.ndarray, null_policy: str):
    """Padded layout of the same mean pool (src/model.py:572-587), per bag."""

    e = np.asarray(embedded, dtype=np.float64)
    ids = np.asarray(indices, dtype=np.int64)
    B, L, D = e.shape
    out = np.zeros((B, D))
    for b in range(B):
        keep = [p for p in range(L) if p < lengths[b] and (null_policy != "exclude" or ids[b, p] != 0)]
        if keep:
            out[b] = e[b, keep].sum(0) / len(keep)
    return out


def pool_rows_backward(indices: np.ndarray, lengths: np.ndarray, grad: np.ndarray, mode: str,
                       null_policy: str) -> np.ndarray:
    """Gradient of pool_rows with respect to every embedded row (autograd of
    the index_add_ + division of src/model.py:564-570): grad[b] * w_i /
    max(counts[b], 1) (mean) or grad[b] * w_i (sum), fp64 [N, dim]."""

    ids = np.asarray(indices, dtype=np.int64)
    g = np.asarray(grad, dtype=np.float64)
    offs = offsets_of(lengths)
    B = offs.size - 1
    seg = np.repeat(np.arange(B), np.diff(offs))
    w = (ids != 0).astype(np.float64) if null_policy == "exclude" else np.ones(ids.size)
    cnt = np.zeros(B)
    np.add.at(cnt, seg, w)
    den = np.maximum(cnt, 1.0) if mode == "mean" else np.ones(B)
    return g[seg] / den[seg][:, None] * w[:, None]


def sequence_gather(weight: np.ndarray, ids: np.ndarray, lengths: np.ndarray, out_len: int,
                    order: str = "oldest_to_newest"):
    """Right-aligned padded gather + mask, brute force, in the reference's
    two steps: ``_right_aligned_sequence`` (src/model.py:2989-3020: lengths
    clamped to [0, out_len], source position p - shift clamped to
    [0, in_len - 1], positions before the shift masked; an empty input gives
    an all-False mask), then for newest_to_oldest the reversal of the valid
    stretch in ``_align_sequence_inputs`` (:3074-3100, source position
    clamped to [0, out_len - 1])."""

    w = np.asarray(weight, dtype=np.float64)
    ids = np.asarray(ids, dtype=np.int64)
    B, in_len = ids.shape
    out = np.zeros((B, out_len, w.shape[1]), dtype=np.float64)
    mask = np.zeros((B, out_len), dtype=bool)
    if out_len == 0 or in_len == 0:
        return out, mask
    aligned = np.zeros_like(out)
    for b in range(B):
        n = min(max(int(lengths[b]), 0), out_len)
        shift = out_len - n
        for p in range(out_len):
            src = min(max(p - shift, 0), in_len - 1)
            mask[b, p] = p >= shift
            aligned[b, p] = w[ids[b, src]] if mask[b, p] else 0.0
    if order == "oldest_to_newest":
        return aligned, mask
    for b in range(B):
        n = min(max(int(lengths[b]), 0), out_len)
        start = out_len - n
        for p in range(out_len):
            src = min(max(out_len - 1 - (p - start), 0), out_len - 1)
            out[b, p] = aligned[b, src] if mask[b, p] else 0.0
    return out, mask


def sequence_positions(ids: np.ndarray, lengths: np.ndarray, out_len: int, order: str = "oldest_to_newest"):
    """Window layout of the right-aligned gather (src/model.py:2989-3100),
    vectorised: ``(mask [B, out_len], src [B, out_len])`` where ``src[b, p]``
    is the input position whose id lands on window position p (valid where
    mask is set: p >= out_len - n_b with n_b = min(max(len_b, 0), out_len),
    and no position when in_len is 0); with rel = p - start, the position is
    min(rel, in_len - 1) oldest first and min(n_b - 1 - rel, in_len - 1)
    newest first, so a length past the input repeats the last element.
    Pinned against the per-position loop of ``sequence_gather``."""

    ids = np.asarray(ids, dtype=np.int64)
    B, in_len = ids.shape
    n = np.minimum(np.maximum(np.asarray(lengths, dtype=np.int64), 0), out_len)
    if in_len == 0:
        n = np.zeros_like(n)
    start = out_len - n
    p = np.arange(out_len, dtype=np.int64)[None, :]
    mask = p >= start[:, None]
    rel = p - start[:, None]
    src = rel if order == "oldest_to_newest" else n[:, None] - 1 - rel
    src = np.minimum(src, max(in_len - 1, 0))
    src = np.where(mask, src, 0)
    return mask, src


def sequence_window(weight: np.ndarray, ids: np.ndarray, lengths: np.ndarray, out_len: int,
                    order: str = "oldest_to_newest"):
    """``sequence_gather`` without the per-position loop, in the weight's own
    dtype (a gather copies rows exactly): ``(out [B, out_len, dim], mask)``."""

    w = np.asarray(weight)
    ids = np.asarray(ids, dtype=np.int64)
    mask, src = sequence_positions(ids, lengths, out_len, order)
    rows = np.take_along_axis(ids, src, axis=1)
    out = w[np.where(mask, rows, 0)]
    out[~mask] = 0
    return out, mask


def sequence_grads(ids: np.ndarray, lengths: np.ndarray, grad: np.ndarray, out_len: int,
                   order: str = "oldest_to_newest", padding_idx: int = 0):
    """(rows, values) of every valid window position whose id is not
    padding: the sparse embedding backward of the window gather (values are
    the window gradient at that position, fp64)."""

    ids = np.asarray(ids, dtype=np.int64)
    mask, src = sequence_positions(ids, lengths, out_len, order)
    rows = np.take_along_axis(ids, src, axis=1)
    keep = mask & (rows != padding_idx)
    return rows[keep], np.asarray(grad)[keep].astype(np.float64)


# ---------------------------------------------------------------- backward --


def per_id_grads(ids: np.ndarray, lengths: np.ndarray | None, grad: np.ndarray, mode: str,
                 null_policy: str, padding_idx: int = 0):
    """(rows, values) of every id that receives a gradient (autograd of the
    pooling, src/model.py:564-570, then the F.embedding sparse backward that
    drops padding_idx).  ``grad`` is [B, dim] (pooled) or [n, dim] (none)."""

    ids = np.asarray(ids, dtype=np.int64)
    grad = np.asarray(grad, dtype=np.float64)
    if mode == "none":
        keep = ids != padding_idx
        return ids[keep], grad[keep]
    offs = offsets_of(lengths)
    seg = np.repeat(np.arange(len(lengths)), np.diff(offs))
    w = np.ones(ids.size) if null_policy != "exclude" else (ids != 0).astype(np.float64)
    cnt = np.zeros(len(lengths))
    np.add.at(cnt, seg, w)
    den = np.maximum(cnt, 1.0) if mode == "mean" else np.ones_like(cnt)
    vals = grad[seg] / den[seg][:, None] * w[:, None]
    keep = (ids != padding_idx) & (w != 0)
    return ids[keep], vals[keep]


def coalesce(rows: np.ndarray, values: np.ndarray):
    """Sorted unique rows and fp64 sums of their values."""

    rows = _c(rows, np.int64)
    vals = _c(values, np.float64)
    n = rows.size
    dim = vals.shape[1] if vals.ndim == 2 else 0
    out_rows = np.empty(max(n, 1), dtype=np.int64)
    out_vals = np.empty((max(n, 1), max(dim, 1)), dtype=np.float64)
    u = _lib().oracle_coalesce(_p(rows), _p(vals), n, dim, _p(out_rows), _p(out_vals))
    return out_rows[:u].copy(), out_vals[:u, :dim].copy()


def unique(ids: np.ndarray):
    ids = np.asarray(ids, dtype=np.int64)
    u, inv, cnt = np.unique(ids, return_inverse=True, return_counts=True)
    return u, inv.reshape(ids.shape), cnt


def rowwise_adagrad(weight: np.ndarray, acc: np.ndarray, rows: np.ndarray, values: np.ndarray,
                    lr: float, eps: float, is_bf16: bool = False):
    """Returns updated copies (weight fp32-widened, acc fp32)."""

    w = _c(weight, np.float32).copy()
    a = _c(acc, np.float32).copy()
    rows = _c(rows, np.int64)
    vals = _c(values, np.float64)
    _lib().oracle_rowwise_adagrad(_p(w), 1 if is_bf16 else 0, w.shape[0], w.shape[1], _p(a), _p(rows),
                                  rows.size, _p(vals), float(lr), float(eps))
    return w, a


def clip_grad_norm(values: list, max_norm: float):
    """_clip_sparse_grad_norm on coalesced values (src/train.py:5745-5826):
    total = sqrt(sum of squared 2-norms) (fp64 here), coef =
    min(max_norm / (total + 1e-6), 1); returns (scaled fp64 copies, total, coef)."""

    vals = [np.asarray(v, dtype=np.float64) for v in values]
    total = float(np.sqrt(sum(float((v * v).sum()) for v in vals)))
    coef = min(max_norm / (total + 1e-6), 1.0)
    return [v * coef for v in vals], total, coef


def sparse_step(features, tables, ids, offsets_rel, out_stride, grad, lr, eps):
    """One fused fwd + bwd + row-wise Adagrad step, in place on the tables.

    features: list of dicts {table, pooling (0/1/2), exclude, ids_off, bag_off,
    num_bags, out_col}; tables: list of dicts {W (fp32 array, updated in place),
    acc (fp32, in place), is_bf16}.  Returns the pooled output [B, out_stride].
    """

    F = len(features)
    T = len(tables)
    i32 = lambda xs: np.asarray(xs, dtype=np.int32)
    i64 = lambda xs: np.asarray(xs, dtype=np.int64)
    table = i32([f["table"] for f in features])
    pooling = i32([f["pooling"] for f in features])
    exclude = i32([f["exclude"] for f in features])
    ids_off = i64([f["ids_off"] for f in features] + [len(ids)])
    bag_off = i64([f["bag_off"] for f in features])
    num_bags = i64([f["num_bags"] for f in features])
    out_col = i64([f["out_col"] for f in features])
    ids = _c(ids, np.int64)
    offs = _c(offsets_rel, np.int64)
    grad = _c(grad, np.float64)
    B = grad.shape[0]
    out = np.zeros((B, out_stride), dtype=np.float64)
    Ws = [t["W"] for t in tables]
    As = [t["acc"] for t in tables]
    for a in Ws + As:
        assert a.dtype == np.float32 and a.flags.c_contiguous
    wptr = (ctypes.c_void_p * T)(*[a.ctypes.data for a in Ws])
    aptr = (ctypes.c_void_p * T)(*[a.ctypes.data for a in As])
    rows = i64([a.shape[0] for a in Ws])
    dims = i32([a.shape[1] for a in Ws])
    bf = i32([1 if t.get("is_bf16") else 0 for t in tables])
    _lib().oracle_sparse_step(
        F, _p(table), _p(pooling), _p(exclude), _p(ids), _p(ids_off), _p(offs), _p(bag_off), _p(num_bags),
        _p(out_col), ctypes.c_int64(out_stride), _p(out), _p(grad), T, ctypes.cast(wptr, _P),
        ctypes.cast(aptr, _P), _p(rows), _p(dims), _p(bf), float(lr), float(eps),
    )
    return out
