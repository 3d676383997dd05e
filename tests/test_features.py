"""Id bucketing and list-feature truncation to CSR bags (host side, no GPU).

The oracle's ``bag_truncate`` restates the reference's Arrow truncation
(src/dataloader.py:8565-8640); it is pinned here by the reference's golden
vectors in Arrow layout, by pyarrow's own list kernels and by the per-row
brute force ``bag_csr``.  The ``mdl_hip::bag_truncate`` op's CPU kernel (the
product's vectorised path) is then checked against the oracle.
"""

import json
from pathlib import Path

import numpy as np
import pyarrow as pa
import pyarrow.compute as pc
import pytest
import torch

import mdl_amd  # noqa: F401  (registers the mdl_hip ops)
from mdl_amd.features import (
    INT64_MAX, INT64_MIN, bag_csr, bag_csr_arrow, bag_csr_tensor, mod_bucket_tensor, pre_hashed_bucket,
    pre_hashed_bucket_tensor,
)
from oracle import oracle as O

GOLD = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())


def _random_lists(rng, rows, max_len, null_rows=0.1, null_elems=0.1):
    out = []
    for _ in range(rows):
        if rng.random() < null_rows:
            out.append(None)
            continue
        n = int(rng.integers(0, max_len + 1))
        vals = rng.integers(-(1 << 63), (1 << 63) - 1, size=n, dtype=np.int64, endpoint=True).tolist()
        out.append([None if rng.random() < null_elems else v for v in vals])
    return out


def _arrow_parts(array):
    offsets = array.offsets.to_numpy(zero_copy_only=False).astype(np.int64)
    raw = pc.fill_null(array.values, 0).to_numpy(zero_copy_only=False).astype(np.int64)
    valid = array.values.is_valid().to_numpy(zero_copy_only=False).astype(np.uint8)
    row_valid = array.is_valid().to_numpy(zero_copy_only=False).astype(np.uint8)
    return offsets, raw, valid, row_valid


@pytest.mark.parametrize("key", ["bag_head_truncation", "bag_tail_truncation"])
def test_oracle_bag_truncate_golden(key):
    g = GOLD[key]
    offsets, raw, valid, row_valid = _arrow_parts(pa.array(g["rows"], type=pa.list_(pa.int64())))
    vals, ok, lengths = O.bag_truncate(offsets, raw, valid, row_valid, g["max_length"], g["truncation"])
    ids, _ = O.bucketize_pre_hashed(vals, g["num_buckets"], ok)
    assert lengths.tolist() == g["expected_lengths"]
    assert ids.tolist() == g["expected_values"]


@pytest.mark.parametrize("truncation", ["head", "tail"])
@pytest.mark.parametrize("max_length", [None, 0, 1, 3, 7])
def test_oracle_bag_truncate_matches_brute_force_and_arrow(truncation, max_length):
    rng = np.random.default_rng(31 + (max_length or 0))
    rows = _random_lists(rng, 300, 9)
    array = pa.array(rows, type=pa.list_(pa.int64()))
    offsets, raw, valid, row_valid = _arrow_parts(array)
    vals, ok, lengths = O.bag_truncate(offsets, raw, valid, row_valid, max_length, truncation)
    flat, bvalid, blengths = bag_csr(rows, max_length=max_length, truncation=truncation)
    assert lengths.tolist() == blengths.tolist()
    assert (vals * ok).tolist() == flat.tolist() and ok.tolist() == bvalid.tolist()
    if truncation == "head" and max_length is not None:
        # pyarrow's own kernels: list_slice, list_value_length (nulls 0), list_flatten
        sliced = pc.list_slice(array, 0, max_length)
        assert pc.fill_null(pc.list_value_length(sliced), 0).to_pylist() == lengths.tolist()
        flat_arrow = pc.list_flatten(sliced)
        assert pc.fill_null(flat_arrow, 0).to_pylist() == (vals * ok).tolist()
        assert flat_arrow.is_valid().to_pylist() == [bool(x) for x in ok]


def test_oracle_bag_truncate_sliced_arrow_array():
    rng = np.random.default_rng(5)
    rows = _random_lists(rng, 120, 6)
    array = pa.array(rows, type=pa.list_(pa.int64())).slice(17, 60)
    offsets, raw, valid, row_valid = _arrow_parts(array)
    assert offsets[0] != 0
    vals, ok, lengths = O.bag_truncate(offsets, raw, valid, row_valid, 4, "tail")
    flat, bvalid, blengths = bag_csr(rows[17:77], max_length=4, truncation="tail")
    assert lengths.tolist() == blengths.tolist() and (vals * ok).tolist() == flat.tolist()


@pytest.mark.parametrize("truncation", ["head", "tail"])
def test_null_row_with_a_non_empty_span(truncation):
    """A null list row whose offsets span elements (Arrow allows it: a mask
    given to ListArray.from_arrays, or a filter, leaves one).  Head
    truncation (list_slice, src/dataloader.py:8576-8577) keeps the row null,
    so its length is 0; the tail rebuild (:8583-8604) reads the raw offsets of
    every row and builds a list array without a validity bitmap, so the row
    keeps its last elements.  Expected values come from pyarrow's kernels
    run through those steps."""

    offsets = pa.array([0, 3, 7, 9], pa.int32())
    values = pa.array([11, 12, 13, 21, 22, 23, 24, 31, 32], pa.int64())
    array = pa.ListArray.from_arrays(offsets, values, mask=pa.array([False, True, False]))
    assert array.null_count == 1 and array.offsets.to_pylist() == [0, 3, 7, 9]
    max_length = 2
    if truncation == "head":
        cut = pc.list_slice(array, 0, max_length)
    else:
        off = array.offsets.to_numpy(zero_copy_only=False).astype(np.int64)
        lengths = off[1:] - off[:-1]
        take = np.minimum(lengths, max_length)
        starts = off[:-1] + (lengths - take)
        idx = np.concatenate([np.arange(a, a + k) for a, k in zip(starts, take)])
        new_offsets = np.concatenate([[0], np.cumsum(take)])
        cut = pa.ListArray.from_arrays(pa.array(new_offsets, pa.int32()), pc.take(array.values, pa.array(idx)))
    exp_lengths = pc.fill_null(pc.list_value_length(cut), 0).to_pylist()
    exp_values = pc.list_flatten(cut).to_pylist()
    assert exp_lengths == ([2, 0, 2] if truncation == "head" else [2, 2, 2])
    offs, raw, valid, row_valid = _arrow_parts(array)
    vals, ok, lengths = O.bag_truncate(offs, raw, valid, row_valid, max_length, truncation)
    assert lengths.tolist() == exp_lengths and vals.tolist() == exp_values and ok.all()
    ids, lens, out_offsets, err = _op_cpu(offs, raw, valid, row_valid, max_length, truncation, "none", 0)
    assert lens.tolist() == exp_lengths and ids[: len(exp_values)].tolist() == exp_values
    assert int(err[0]) == 0
    # without truncation a null row has length 0 (list_value_length, nulls as 0)
    vals, ok, lengths = O.bag_truncate(offs, raw, valid, row_valid, None, truncation)
    assert lengths.tolist() == [3, 0, 2]
    ids, lens, _, _ = _op_cpu(offs, raw, valid, row_valid, None, truncation, "none", 0)
    assert lens.tolist() == [3, 0, 2]


def _op_cpu(offsets, raw, valid, row_valid, max_length, truncation, bucket, nb, validate=True):
    t = lambda a, dt=torch.int64: None if a is None else torch.from_numpy(np.asarray(a)).to(dt)  # noqa: E731
    return torch.ops.mdl_hip.bag_truncate(t(raw), t(offsets), t(valid, torch.uint8), t(row_valid, torch.uint8),
                                          -1 if max_length is None else max_length, truncation, bucket, nb,
                                          validate)


@pytest.mark.parametrize("bucket,nb", [("none", 0), ("pre_hashed", 1 << 20), ("mod", 1_000_003)])
@pytest.mark.parametrize("truncation", ["head", "tail"])
def test_bag_truncate_cpu_kernel_matches_oracle(bucket, nb, truncation):
    rng = np.random.default_rng(77)
    array = pa.array(_random_lists(rng, 500, 12), type=pa.list_(pa.int64()))
    offsets, raw, valid, row_valid = _arrow_parts(array)
    raw[raw == 0] = 1  # zeros are the error case, tested below
    ids, lengths, out_offsets, err = _op_cpu(offsets, raw, valid, row_valid, 5, truncation, bucket, nb)
    vals, ok, ref_lengths = O.bag_truncate(offsets, raw, valid, row_valid, 5, truncation)
    if bucket == "none":
        ref = vals * ok
    elif bucket == "pre_hashed":
        ref, _ = O.bucketize_pre_hashed(vals, nb, ok)
    else:
        ref = O.bucketize_mod(vals, nb, ok)
    total = int(ref_lengths.sum())
    assert lengths.tolist() == ref_lengths.tolist()
    assert out_offsets.tolist() == O.offsets_of(ref_lengths).tolist()
    assert ids[:total].tolist() == ref.tolist() and not ids[total:].any()
    assert int(err[0]) == 0


def test_bag_truncate_cpu_kernel_counts_zeros_and_bad_offsets():
    offsets = np.array([0, 2, 5, 5], dtype=np.int64)
    raw = np.array([0, 3, 4, 0, 6], dtype=np.int64)
    valid = np.array([1, 1, 1, 0, 1], dtype=np.uint8)
    _, _, _, err = _op_cpu(offsets, raw, valid, None, None, "head", "pre_hashed", 8)
    assert int(err[0]) == 1  # the null zero is not counted
    _, _, _, err = _op_cpu(offsets, raw, valid, None, None, "head", "pre_hashed", 8, validate=False)
    assert int(err[0]) == 0
    bad = np.array([0, 7, 3, -1], dtype=np.int64)  # past the values, decreasing, negative
    ids, lengths, out_offsets, err = _op_cpu(bad, raw, None, None, None, "tail", "none", 0)
    assert lengths.tolist() == [5, 0, 0] and int(err[0]) == 3
    assert ids.tolist() == raw.tolist()


def test_bag_csr_tensor_errors_and_capacity_form():
    raw = torch.tensor([5, 0, 7], dtype=torch.int64)
    offsets = torch.tensor([0, 2, 3], dtype=torch.int64)
    with pytest.raises(ValueError, match="non-null zero"):
        bag_csr_tensor(raw, offsets, bucket="pre_hashed", num_buckets=8)
    with pytest.raises(ValueError, match="offsets outside"):
        bag_csr_tensor(raw, torch.tensor([0, 4, 3], dtype=torch.int64))
    out = bag_csr_tensor(raw, offsets, max_length=1, truncation="tail", exact=False)
    assert out["values"].tolist() == [0, 7, 0] and out["offsets"].tolist() == [0, 1, 2]
    assert int(out["errors"][0]) == 0


@pytest.mark.parametrize("key", ["bag_head_truncation", "bag_tail_truncation"])
def test_bag_csr_arrow_golden_cpu(key):
    g = GOLD[key]
    out = bag_csr_arrow(pa.array(g["rows"], type=pa.list_(pa.int64())), max_length=g["max_length"],
                        truncation=g["truncation"], bucket="pre_hashed", num_buckets=g["num_buckets"])
    assert out["values"].tolist() == g["expected_values"]
    assert out["lengths"].tolist() == g["expected_lengths"]


def test_bag_truncate_opcheck_cpu():
    rng = np.random.default_rng(3)
    array = pa.array(_random_lists(rng, 40, 6), type=pa.list_(pa.int64()))
    offsets, raw, valid, row_valid = _arrow_parts(array)
    raw[raw == 0] = 1
    args = (torch.from_numpy(raw), torch.from_numpy(offsets), torch.from_numpy(valid), torch.from_numpy(row_valid),
            3, "tail", "pre_hashed", 64, True)
    torch.library.opcheck(torch.ops.mdl_hip.bag_truncate.default, args)


def test_pre_hashed_bucket_scalar_follows_the_reference():
    """The scalar API on the reference's golden values and errors
    (tests/test_direct_id.py:183-189, src/features.py:360-376)."""

    g = GOLD["pre_hashed_scalar"]
    for raw, want in g["cases"]:
        assert pre_hashed_bucket(raw, g["num_buckets"]) == want
    assert pre_hashed_bucket(1, 8) == 2 and pre_hashed_bucket(7, 8) == 8 and pre_hashed_bucket(9, 8) == 2
    with pytest.raises(ValueError, match="must not be zero"):
        pre_hashed_bucket(0, 8)
    with pytest.raises(TypeError, match="must be an int64"):
        pre_hashed_bucket(True, 8)
    with pytest.raises(TypeError, match="must be an int64"):
        pre_hashed_bucket(3.0, 8)
    with pytest.raises(ValueError, match="outside signed int64"):
        pre_hashed_bucket(1 << 63, 8)
    with pytest.raises(ValueError, match="power of two"):
        pre_hashed_bucket(5, 6)


def test_bucket_tensors_on_the_host_follow_the_reference():
    """The tensor forms on CPU tensors (the op's CPU kernel), on the golden
    columns of tests/test_direct_id.py:191-240 and, for the mod rule, on
    random int64 values against Python's floor-mod (src/benchmark.py:1246-1250)."""

    g = GOLD["pre_hashed_column_with_nulls"]
    valid = torch.tensor([v is not None for v in g["raw"]])
    raw = torch.tensor([0 if v is None else v for v in g["raw"]], dtype=torch.int64)
    assert pre_hashed_bucket_tensor(raw, g["num_buckets"], valid=valid).tolist() == g["expected"]
    z = GOLD["pre_hashed_zero_unvalidated"]
    zraw = torch.tensor(z["raw"], dtype=torch.int64)
    with pytest.raises(ValueError, match="non-null zero"):
        pre_hashed_bucket_tensor(zraw, z["num_buckets"], name="item_hash")
    assert pre_hashed_bucket_tensor(zraw, z["num_buckets"], validate_nonzero=False).tolist() == z["expected"]
    # a null zero is not an error
    assert pre_hashed_bucket_tensor(zraw, 8, valid=torch.tensor([True, False])).tolist() == [2, 0]

    rng = np.random.default_rng(9)
    vals = rng.integers(INT64_MIN, INT64_MAX, size=2000, dtype=np.int64, endpoint=True)
    vals[:4] = [INT64_MIN, INT64_MAX, 0, 1]
    for n in (2, 3, 1_000_000, 999_999_937, (1 << 62) + 1):
        got = mod_bucket_tensor(torch.from_numpy(vals), n).tolist()
        assert got == [1 + ((int(v) - 1) % (n - 1)) for v in vals], n
    assert mod_bucket_tensor(torch.from_numpy(vals), 1).tolist() == [0] * len(vals)
