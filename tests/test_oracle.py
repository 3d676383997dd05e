"""Pins the CPU oracle (oracle/) before it is trusted as the checker.

Each check compares the oracle with something independent of it: the
reference tests' own golden vectors (tests/golden/reference_vectors.json),
Python's arbitrary-precision integer arithmetic, or a PyTorch library routine
run on the CPU (F.embedding_bag, sparse coalesce, torch.unique, autograd).
"""

import json
import pathlib

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as O
from mdl_amd.features import bag_csr

GOLD = json.loads((pathlib.Path(__file__).parent / "golden" / "reference_vectors.json").read_text())
INT64_MIN = -(1 << 63)
INT64_MAX = (1 << 63) - 1


def _raw_with_nulls(values):
    raw = np.array([0 if v is None else v for v in values], dtype=np.int64)
    valid = np.array([0 if v is None else 1 for v in values], dtype=np.uint8)
    return raw, valid


def test_pre_hashed_golden_scalars():
    g = GOLD["pre_hashed_scalar"]
    raw = np.array([c[0] for c in g["cases"]], dtype=np.int64)
    out, zeros = O.bucketize_pre_hashed(raw, g["num_buckets"])
    assert out.tolist() == [c[1] for c in g["cases"]]
    assert zeros == 0
    _, zeros = O.bucketize_pre_hashed(np.array([0], dtype=np.int64), 8)
    assert zeros == 1


def test_pre_hashed_golden_column_with_nulls():
    for key in ("pre_hashed_column_with_nulls", "pre_hashed_zero_unvalidated"):
        g = GOLD[key]
        raw, valid = _raw_with_nulls(g["raw"])
        out, _ = O.bucketize_pre_hashed(raw, g["num_buckets"], valid)
        assert out.tolist() == g["expected"]


def test_pre_hashed_matches_python_bit_arithmetic():
    rng = np.random.default_rng(1)
    raw = rng.integers(INT64_MIN, INT64_MAX, size=5000, dtype=np.int64, endpoint=True)
    raw[:4] = [INT64_MIN, INT64_MAX, -1, 1]
    for buckets in (1, 2, 8, 1 << 20, 1 << 40):
        out, _ = O.bucketize_pre_hashed(raw, buckets)
        expect = [(int(v) & (buckets - 1)) + 1 for v in raw]
        assert out.tolist() == expect


def test_mod_matches_python_floor_mod():
    rng = np.random.default_rng(2)
    raw = rng.integers(INT64_MIN, INT64_MAX, size=5000, dtype=np.int64, endpoint=True)
    raw[:5] = [INT64_MIN, INT64_MAX, 0, 1, -1]
    for n in (2, 3, 1_000_000, 999_999_937):
        out = O.bucketize_mod(raw, n)
        assert out.tolist() == [1 + ((int(v) - 1) % (n - 1)) for v in raw]


@pytest.mark.parametrize("key", ["bag_head_truncation", "bag_tail_truncation", "pre_hashed_sequence_head"])
def test_bag_csr_golden(key):
    g = GOLD[key]
    flat, valid, lengths = bag_csr(g["rows"], max_length=g["max_length"], truncation=g["truncation"])
    ids, _ = O.bucketize_pre_hashed(flat, g["num_buckets"], valid)
    assert lengths.tolist() == g["expected_lengths"]
    if "expected_values" in g:
        assert ids.tolist() == g["expected_values"]
    else:  # right-padded sequence layout
        width = max(g["expected_lengths"])
        padded = np.zeros((len(lengths), width), dtype=np.int64)
        offs = O.offsets_of(lengths)
        for b in range(len(lengths)):
            padded[b, : lengths[b]] = ids[offs[b]: offs[b + 1]]
        assert padded.tolist() == g["expected_padded"]


def test_pool_golden_null_policies():
    g = GOLD["mean_pool_null_policies"]
    table = np.arange(16, dtype=np.float32).reshape(16, 1)  # row i holds the value i
    ex, _ = O.pool(table, np.array(g["indices"]), np.array(g["lengths"]), "mean", "exclude")
    inc, _ = O.pool(table, np.array(g["indices"]), np.array(g["lengths"]), "mean", "include_as_padding")
    np.testing.assert_allclose(ex, g["expected_exclude"], rtol=1e-12)
    np.testing.assert_allclose(inc, g["expected_include_as_padding"], rtol=1e-12)


@pytest.mark.parametrize("mode", ["sum", "mean"])
def test_pool_matches_torch_embedding_bag(mode):
    rng = np.random.default_rng(3)
    rows, dim, B = 50, 7, 64
    W = rng.standard_normal((rows, dim)).astype(np.float32)
    lengths = rng.integers(0, 9, size=B)
    ids = rng.integers(0, rows, size=int(lengths.sum()))
    ids[::5] = 0
    offs = O.offsets_of(lengths)
    # "exclude": padding id 0 leaves the sum and the mean's count
    got, _ = O.pool(W, ids, lengths, mode, "exclude")
    ref = F.embedding_bag(torch.from_numpy(ids), torch.from_numpy(W).double(), torch.from_numpy(offs[:-1]),
                          mode=mode, padding_idx=0)
    np.testing.assert_allclose(got, ref.numpy(), rtol=1e-12, atol=1e-12)
    # "include_as_padding": every id (row 0 included) counts
    got, _ = O.pool(W, ids, lengths, mode, "include_as_padding")
    ref = F.embedding_bag(torch.from_numpy(ids), torch.from_numpy(W).double(), torch.from_numpy(offs[:-1]),
                          mode=mode)
    np.testing.assert_allclose(got, ref.numpy(), rtol=1e-12, atol=1e-12)


def test_pool_rows_golden_flat_and_padded():
    g = GOLD["mean_pool_null_policies"]
    idx = np.array(g["indices"])
    emb = idx.astype(np.float64)[:, None]  # the embedded row of an id holds the id
    ex, _ = O.pool_rows(emb, idx, np.array(g["lengths"]), "mean", "exclude")
    inc, _ = O.pool_rows(emb, idx, np.array(g["lengths"]), "mean", "include_as_padding")
    np.testing.assert_allclose(ex, g["expected_exclude"], rtol=1e-12)
    np.testing.assert_allclose(inc, g["expected_include_as_padding"], rtol=1e-12)
    p = GOLD["mean_pool_padded"]
    pidx = np.array(p["indices"])
    pad = O.pool_rows_padded(pidx.astype(np.float64)[..., None], pidx, np.array(p["lengths"]), "exclude")
    np.testing.assert_allclose(pad, p["expected_exclude"], rtol=1e-12)


@pytest.mark.parametrize("policy", ["exclude", "include_as_padding"])
@pytest.mark.parametrize("mode", ["sum", "mean"])
def test_pool_rows_match_embedding_bag_and_autograd(mode, policy):
    """Rows pooled by position = F.embedding_bag over arange(N) with the null
    weights as per-sample weights; the backward = its autograd."""

    rng = np.random.default_rng(11)
    B, dim = 48, 6
    lengths = rng.integers(0, 7, size=B)
    n = int(lengths.sum())
    ids = rng.integers(0, 5, size=n)  # many nulls
    emb = torch.from_numpy(rng.standard_normal((n, dim))).requires_grad_(True)
    offs = O.offsets_of(lengths)
    w = (ids != 0).astype(np.float64) if policy == "exclude" else np.ones(n)
    cnt = np.add.reduceat(np.append(w, 0.0), offs[:-1])[:B] * (np.diff(offs) > 0)
    den = np.maximum(cnt, 1.0) if mode == "mean" else np.ones(B)
    seg = np.repeat(np.arange(B), np.diff(offs))
    psw = torch.from_numpy(w / den[seg])
    ref = F.embedding_bag(torch.arange(n), emb, torch.from_numpy(offs[:-1]), mode="sum", per_sample_weights=psw)
    got, got_cnt = O.pool_rows(emb.detach().numpy(), ids, lengths, mode, policy)
    np.testing.assert_allclose(got, ref.detach().numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(got_cnt, cnt, rtol=0, atol=0)
    g = rng.standard_normal((B, dim))
    ref.backward(torch.from_numpy(g))
    back = O.pool_rows_backward(ids, lengths, g, mode, policy)
    np.testing.assert_allclose(back, emb.grad.numpy(), rtol=1e-12, atol=1e-12)
    # adjoint identity of the linear map E -> pool(E)
    E = rng.standard_normal((n, dim))
    lhs = float((O.pool_rows(E, ids, lengths, mode, policy)[0] * g).sum())
    rhs = float((E * back).sum())
    assert abs(lhs - rhs) <= 1e-10 * max(1.0, abs(lhs))


def test_pool_rows_padded_equals_flat():
    rng = np.random.default_rng(12)
    B, L, dim = 20, 5, 3
    lengths = rng.integers(0, L + 1, size=B)
    idx = rng.integers(0, 4, size=(B, L))
    emb = rng.standard_normal((B, L, dim))
    for policy in ("exclude", "include_as_padding"):
        pad = O.pool_rows_padded(emb, idx, lengths, policy)
        flat_e = np.concatenate([emb[b, : lengths[b]] for b in range(B)])
        flat_i = np.concatenate([idx[b, : lengths[b]] for b in range(B)])
        flat, _ = O.pool_rows(flat_e, flat_i, lengths, "mean", policy)
        np.testing.assert_allclose(pad, flat, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("policy", ["exclude", "include_as_padding"])
@pytest.mark.parametrize("mode", ["sum", "mean", "none"])
def test_per_id_grads_match_autograd(mode, policy):
    """Coalesced per-id gradients equal torch autograd's dense weight grad."""

    rng = np.random.default_rng(4)
    rows, dim, B = 30, 5, 40
    W = torch.from_numpy(rng.standard_normal((rows, dim))).double().requires_grad_(True)
    lengths = rng.integers(0, 6, size=B)
    ids = rng.integers(0, rows, size=int(lengths.sum()))
    ids[::4] = 0
    offs = O.offsets_of(lengths)
    if mode == "none":
        out = F.embedding(torch.from_numpy(ids), W, padding_idx=0)
        g = rng.standard_normal(out.shape)
    else:
        pad = 0 if policy == "exclude" else None
        out = F.embedding_bag(torch.from_numpy(ids), W, torch.from_numpy(offs[:-1]), mode=mode,
                              padding_idx=pad)
        if policy == "include_as_padding":
            # the reference never propagates into padding row 0 (F.embedding padding_idx)
            pass
        g = rng.standard_normal(out.shape)
    out.backward(torch.from_numpy(g))
    dense = W.grad.numpy().copy()
    if policy == "include_as_padding":
        dense[0] = 0.0
    r, v = O.per_id_grads(ids, None if mode == "none" else lengths, g, mode, policy)
    cr, cv = O.coalesce(r, v)
    expect_rows = np.nonzero(np.abs(dense).sum(1))[0]
    assert set(expect_rows.tolist()) <= set(cr.tolist())
    full = np.zeros_like(dense)
    full[cr] = cv
    np.testing.assert_allclose(full, dense, rtol=1e-12, atol=1e-12)


def test_coalesce_and_unique_match_torch():
    rng = np.random.default_rng(5)
    n, dim = 3000, 3
    rows = rng.zipf(1.3, size=n) % 97
    vals = rng.standard_normal((n, dim))
    cr, cv = O.coalesce(rows, vals)
    t = torch.sparse_coo_tensor(torch.from_numpy(rows)[None], torch.from_numpy(vals), (97, dim)).coalesce()
    assert cr.tolist() == t.indices()[0].tolist()
    np.testing.assert_allclose(cv, t.values().numpy(), rtol=1e-12, atol=1e-12)
    u, inv, cnt = O.unique(rows)
    tu, tinv, tcnt = torch.unique(torch.from_numpy(rows), sorted=True, return_inverse=True, return_counts=True)
    assert u.tolist() == tu.tolist() and inv.tolist() == tinv.tolist() and cnt.tolist() == tcnt.tolist()


def test_rowwise_adagrad_golden_mean_not_sum():
    g = GOLD["rowwise_adagrad_mean_not_sum"]
    W = np.zeros(g["shape"], dtype=np.float32)
    acc = np.full(g["shape"][0], g["acc0"], dtype=np.float32)
    W2, acc2 = O.rowwise_adagrad(W, acc, np.array(g["rows"]), np.array(g["values"]), g["lr"], g["eps"])
    for r, a in g["expected_acc"].items():
        assert abs(acc2[int(r)] - a) < 1e-6
    for r, w in g["expected_neg_weight"].items():
        np.testing.assert_allclose(-W2[int(r)], w, atol=g["atol"])


def test_rowwise_adagrad_golden_duplicates_via_coalesce():
    g = GOLD["rowwise_adagrad_duplicates_coalesce"]
    rows, vals = O.coalesce(np.array(g["rows"]), np.array(g["values"], dtype=np.float64))
    W = np.zeros(g["shape"], dtype=np.float32)
    acc = np.zeros(g["shape"][0], dtype=np.float32)
    _, acc2 = O.rowwise_adagrad(W, acc, rows, vals, g["lr"], g["eps"])
    assert abs(acc2[3] - g["expected_acc"]["3"]) < 1e-6
    assert int((acc2 != 0).sum()) == g["expected_nonzero_acc_rows"]


def test_rowwise_adagrad_golden_bf16_untouched():
    g = GOLD["rowwise_adagrad_bf16_untouched"]
    W = np.array(g["weight"], dtype=np.float32)
    rows, vals = O.coalesce(np.array(g["rows"]), np.array(g["values"], dtype=np.float64))
    acc = np.zeros(W.shape[0], dtype=np.float32)
    W2, acc2 = O.rowwise_adagrad(W, acc, rows, vals, g["lr"], g["eps"], is_bf16=True)
    for r in g["untouched_rows"]:
        assert np.array_equal(W2[r], W[r])
    assert not np.array_equal(W2[1], W[1])
    assert abs(acc2[1] - g["expected_acc_row1"]) < 1e-6
    assert np.array_equal(W2, O.round_bf16(W2))  # stored values are bf16


def test_rowwise_adagrad_shard_equals_full_table():
    g = GOLD["rowwise_adagrad_shard_vs_full"]
    rng = np.random.default_rng(0)
    full = rng.standard_normal((8, 4)).astype(np.float32)
    rows = np.array(g["rows"])
    vals = np.array(g["values"], dtype=np.float64)
    Wf, af = O.rowwise_adagrad(full, np.zeros(8, np.float32), rows, vals, g["lr"], g["eps"])
    for rank in range(2):  # cyclic owners: global row r lives on rank r % 2 at local row r // 2
        own = rows % 2 == rank
        Ws, as_ = O.rowwise_adagrad(full[rank::2], np.zeros(4, np.float32), rows[own] // 2, vals[own],
                                    g["lr"], g["eps"])
        np.testing.assert_allclose(Ws, Wf[rank::2], atol=1e-6)
        np.testing.assert_allclose(as_, af[rank::2], atol=1e-6)


def test_rowwise_adagrad_matches_reference_formula_in_torch():
    """Same update from torch ops on the CPU (mean of squares, eps after sqrt)."""

    rng = np.random.default_rng(6)
    W = rng.standard_normal((20, 6)).astype(np.float32)
    acc = rng.random(20).astype(np.float32)
    rows = np.array([1, 4, 7, 19])
    vals = rng.standard_normal((4, 6))
    W2, a2 = O.rowwise_adagrad(W, acc, rows, vals, 0.05, 1e-8)
    tw = torch.from_numpy(W).double()
    ta = torch.from_numpy(acc).double()
    tv = torch.from_numpy(vals)
    ta[rows] += tv.square().mean(1)
    tw[rows] -= 0.05 * tv / (ta[rows].sqrt() + 1e-8)[:, None]
    np.testing.assert_allclose(W2, tw.numpy(), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(a2, ta.numpy(), rtol=1e-6)


def test_sequence_gather_closed_forms():
    W = np.arange(10, dtype=np.float32)[:, None] * np.ones((1, 2), np.float32)
    out, mask = O.sequence_gather(W, np.array([[8, 1], [0, 0]]), np.array([2, 0]), 2)
    assert mask.tolist() == [[True, True], [False, False]]
    assert out[0, :, 0].tolist() == [8.0, 1.0] and out[1].sum() == 0
    out, mask = O.sequence_gather(W, np.array([[3, 4, 0]]), np.array([2]), 3)
    assert mask.tolist() == [[False, True, True]] and out[0, :, 0].tolist() == [0.0, 3.0, 4.0]
    out, _ = O.sequence_gather(W, np.array([[3, 4, 0]]), np.array([2]), 3, "newest_to_oldest")
    assert out[0, :, 0].tolist() == [0.0, 4.0, 3.0]


def test_sequence_gather_length_past_the_input():
    """A length past the input width (hand-traced through
    src/model.py:3011-3016 and :3091-3099): input [e0, e1], length 3, width 4
    gives [0, e0, e1, e1] with mask [F, T, T, T]; newest first the valid
    stretch reverses to [0, e1, e1, e0].  An empty input masks everything
    (:3000-3009)."""

    W = np.arange(10, dtype=np.float32)[:, None] * np.ones((1, 2), np.float32)
    ids = np.array([[5, 7]])
    out, mask = O.sequence_gather(W, ids, np.array([3]), 4)
    assert mask.tolist() == [[False, True, True, True]]
    assert out[0, :, 0].tolist() == [0.0, 5.0, 7.0, 7.0]
    out, mask = O.sequence_gather(W, ids, np.array([3]), 4, "newest_to_oldest")
    assert mask.tolist() == [[False, True, True, True]]
    assert out[0, :, 0].tolist() == [0.0, 7.0, 7.0, 5.0]
    out, mask = O.sequence_gather(W, np.zeros((2, 0), np.int64), np.array([3, 0]), 4)
    assert not mask.any() and out.sum() == 0
    for order in ("oldest_to_newest", "newest_to_oldest"):
        m, src = O.sequence_positions(ids, np.array([3]), 4, order)
        ref, rmask = O.sequence_gather(W, ids, np.array([3]), 4, order)
        assert np.array_equal(m, rmask)
        assert np.array_equal(np.where(m, W[np.take_along_axis(ids, src, 1)][..., 0], 0), ref[..., 0])


def _reference_window_torch(emb: torch.Tensor, lengths: torch.Tensor, out_len: int, order: str):
    """The reference's window steps written with torch ops, for pinning: the
    gather/clamp/mask of src/model.py:2998-3020, then the reversal of
    :3091-3099 for newest_to_oldest."""

    B, L, D = emb.shape
    if L == 0:
        return emb.new_zeros(B, out_len, D), torch.zeros(B, out_len, dtype=torch.bool)
    n = lengths.clamp(min=0, max=out_len)
    pos = torch.arange(out_len).view(1, -1)
    shifts = (out_len - n).view(-1, 1)
    src = (pos - shifts).clamp(min=0, max=L - 1)
    mask = pos >= shifts
    aligned = emb.gather(1, src.unsqueeze(-1).expand(-1, -1, D)) * mask.unsqueeze(-1).to(emb.dtype)
    if order == "oldest_to_newest":
        return aligned, mask
    starts = (out_len - n).view(-1, 1)
    src2 = (out_len - 1 - (pos - starts)).clamp(min=0, max=out_len - 1)
    rev = aligned.gather(1, src2.unsqueeze(-1).expand(-1, -1, D))
    return rev * mask.unsqueeze(-1).to(rev.dtype), mask


@pytest.mark.parametrize("order", ["oldest_to_newest", "newest_to_oldest"])
def test_sequence_gather_matches_reference_steps_in_torch(order):
    """The oracle's window against the reference's torch steps (restated in
    the test with library gathers), over lengths past the input and the
    window, zero and negative lengths."""

    rng = np.random.default_rng(23)
    W = rng.standard_normal((40, 3))
    B, L_in = 10, 6
    ids = rng.integers(0, 40, size=(B, L_in))
    lengths = np.array([0, 1, 3, 6, 8, -2, 5, 12, 2, 7])
    emb = torch.from_numpy(W)[torch.from_numpy(ids)]
    for out_len in (1, 4, 6, 9):
        ref, rmask = _reference_window_torch(emb, torch.from_numpy(lengths), out_len, order)
        out, mask = O.sequence_gather(W, ids, lengths, out_len, order)
        assert np.array_equal(mask, rmask.numpy())
        assert np.array_equal(out, ref.numpy())


@pytest.mark.parametrize("order", ["oldest_to_newest", "newest_to_oldest"])
def test_sequence_window_equals_per_position_gather(order):
    """The vectorised window (used at full config sizes) against the
    per-position definition, with lengths past both the input and the
    window, zero and negative lengths."""

    rng = np.random.default_rng(21)
    W = rng.standard_normal((50, 3)).astype(np.float32)
    B, L_in = 9, 7
    ids = rng.integers(0, 50, size=(B, L_in))
    lengths = np.array([0, 1, 3, 7, 9, -2, 5, 6, 2])
    for out_len in (1, 4, 7, 10):
        ref, rmask = O.sequence_gather(W, ids, lengths, out_len, order)
        out, mask = O.sequence_window(W, ids, lengths, out_len, order)
        assert out.dtype == np.float32
        assert np.array_equal(mask, rmask)
        assert np.array_equal(out.astype(np.float64), ref)


@pytest.mark.parametrize("order", ["oldest_to_newest", "newest_to_oldest"])
def test_sequence_grads_match_embedding_autograd(order):
    """Window gradients scattered to rows equal the autograd of
    F.embedding(padding_idx=0) followed by the right-aligned window gather
    (library routine, CPU)."""

    rng = np.random.default_rng(22)
    rows, dim, B, L_in = 30, 4, 6, 8
    ids = rng.integers(0, rows, size=(B, L_in))
    ids[:, 1] = 0  # padding inside sequences
    lengths = np.array([0, 2, 8, 5, 11, 1])
    # width 10: lengths 11 and 8 < 10 < 11 reach past the input (repeated last element)
    for out_len in (6, 10):
        grad = rng.standard_normal((B, out_len, dim))
        r, v = O.sequence_grads(ids, lengths, grad, out_len, order)
        dense = np.zeros((rows, dim))
        np.add.at(dense, r, v)
        W = torch.zeros((rows, dim), dtype=torch.float64, requires_grad=True)
        emb = torch.nn.functional.embedding(torch.from_numpy(ids), W, padding_idx=0)
        win, _ = _reference_window_torch(emb, torch.from_numpy(lengths), out_len, order)
        (win * torch.from_numpy(grad)).sum().backward()
        np.testing.assert_allclose(dense, W.grad.numpy(), rtol=1e-12, atol=1e-12)


def test_sparse_step_equals_composition():
    rng = np.random.default_rng(7)
    B = 16
    dims = [4, 8]
    tables = [
        {"W": rng.standard_normal((40, dims[0])).astype(np.float32), "acc": np.zeros(40, np.float32)},
        {"W": rng.standard_normal((25, dims[1])).astype(np.float32), "acc": np.zeros(25, np.float32)},
    ]
    W0 = [t["W"].copy() for t in tables]
    lengths = rng.integers(0, 5, size=B)
    bag_ids = rng.integers(0, 40, size=int(lengths.sum()))
    single = rng.integers(0, 25, size=B)
    ids = np.concatenate([bag_ids, single])
    feats = [
        {"table": 0, "pooling": 2, "exclude": 1, "ids_off": 0, "bag_off": 0, "num_bags": B, "out_col": 0},
        {"table": 1, "pooling": 0, "exclude": 0, "ids_off": len(bag_ids), "bag_off": 0, "num_bags": 0,
         "out_col": dims[0]},
    ]
    stride = sum(dims)
    grad = rng.standard_normal((B, stride))
    out = O.sparse_step(feats, tables, ids, O.offsets_of(lengths), stride, grad, 0.1, 1e-8)
    pooled, _ = O.pool(W0[0], bag_ids, lengths, "mean", "exclude")
    np.testing.assert_allclose(out[:, :4], pooled, rtol=1e-12)
    np.testing.assert_allclose(out[:, 4:], O.gather(W0[1], single), rtol=1e-12)
    r0, v0 = O.per_id_grads(bag_ids, lengths, grad[:, :4], "mean", "exclude")
    r0, v0 = O.coalesce(r0, v0)
    Wexp, _ = O.rowwise_adagrad(W0[0], np.zeros(40, np.float32), r0, v0, 0.1, 1e-8)
    np.testing.assert_allclose(tables[0]["W"], Wexp, rtol=1e-6, atol=1e-7)
    r1, v1 = O.per_id_grads(single, None, grad[:, 4:], "none", "include_as_padding")
    r1, v1 = O.coalesce(r1, v1)
    Wexp, _ = O.rowwise_adagrad(W0[1], np.zeros(25, np.float32), r1, v1, 0.1, 1e-8)
    np.testing.assert_allclose(tables[1]["W"], Wexp, rtol=1e-6, atol=1e-7)


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(8)
    x = (rng.standard_normal(10000) * 10.0 ** rng.integers(-5, 5, 10000)).astype(np.float32)
    ours = O.f32_to_bf16_bits(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)


@pytest.mark.parametrize("max_norm", [0.5, 1.0, 1e6])
def test_clip_grad_norm_matches_torch_clip_grad_norm(max_norm):
    rng = np.random.default_rng(31)
    vals = [rng.standard_normal((int(rng.integers(1, 40)), 8)) * 0.1 for _ in range(5)]
    params = [torch.nn.Parameter(torch.zeros(v.shape, dtype=torch.float64)) for v in vals]
    for p, v in zip(params, vals):
        p.grad = torch.from_numpy(v.copy())
    ref_norm = torch.nn.utils.clip_grad_norm_(params, max_norm)
    got, total, coef = O.clip_grad_norm(vals, max_norm)
    assert abs(total - float(ref_norm)) <= 1e-12 * max(1.0, total)
    for g, p in zip(got, params):
        np.testing.assert_allclose(g, p.grad.numpy(), rtol=1e-12, atol=0)
    if max_norm >= total:
        assert coef == 1.0
        for g, v in zip(got, vals):
            np.testing.assert_array_equal(g, v)


def test_torch_cpu_path_equals_c_oracle():
    """The PyTorch CPU restatement of the reference step (the bench's CPU
    baseline) and the C oracle agree on pooled outputs and updated tables."""

    from oracle import torch_path as TP

    rng = np.random.default_rng(31)
    B = 40
    rows = [60, 25, 90]
    dims = [4, 8, 16]
    pools = ["mean", "none", "sum"]
    W = [rng.standard_normal((r, d)).astype(np.float32) for r, d in zip(rows, dims)]
    for w in W:
        w[0] = 0
    ids, lens = [], []
    for t, p in enumerate(pools):
        if p == "none":
            ids.append(rng.integers(0, rows[t], size=B))
            lens.append(None)
        else:
            ln = rng.integers(0, 6, size=B)
            ids.append(rng.integers(0, rows[t], size=int(ln.sum())))
            lens.append(ln)
    grad = rng.standard_normal((B, sum(dims)))
    cols = np.concatenate([[0], np.cumsum(dims)[:-1]])
    step = TP.TorchStep([torch.from_numpy(w.copy()) for w in W], [torch.full((r,), 0.5) for r in rows],
                        [TP.Feature(t, p) for t, p in enumerate(pools)])
    outs = step.step([torch.from_numpy(x) for x in ids], [None if ln is None else torch.from_numpy(ln) for ln in lens],
                     [torch.from_numpy(grad[:, c: c + d]).float() for c, d in zip(cols, dims)], 0.05, 1e-8)
    feats, offs, bag_off, ids_off = [], [], 0, 0
    for t, (p, x, ln) in enumerate(zip(pools, ids, lens)):
        feats.append({"table": t, "pooling": {"none": 0, "sum": 1, "mean": 2}[p], "exclude": 1, "ids_off": ids_off,
                      "bag_off": bag_off, "num_bags": 0 if ln is None else B, "out_col": int(cols[t])})
        if ln is not None:
            o = O.offsets_of(ln)
            offs.append(o)
            bag_off += len(o)
        ids_off += x.size
    tables = [{"W": w.copy(), "acc": np.full(r, 0.5, np.float32)} for w, r in zip(W, rows)]
    grad32 = grad.astype(np.float32).astype(np.float64)
    ref = O.sparse_step(feats, tables, np.concatenate(ids), np.concatenate(offs), sum(dims), grad32, 0.05, 1e-8)
    for t in range(3):
        np.testing.assert_allclose(outs[t].numpy(), ref[:, cols[t]: cols[t] + dims[t]], rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(step.params[t].detach().numpy(), tables[t]["W"], rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(step.accs[t].numpy(), tables[t]["acc"], rtol=1e-5, atol=1e-6)
