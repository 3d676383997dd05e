"""GPU parity of every libmdl_hip kernel against the CPU oracle.

Integer work (bucketing, offsets, sort, unique, coalesced rows) must match
bit for bit; floating point within 1e-5 relative for fp32 storage and 1e-2
relative for bf16 storage (fp32 accumulation), the tolerances the path's
specification states.  Every case prints its name and shape before it runs.
"""

import sys

import numpy as np
import pytest
import torch

from mdl_amd import _lib, ops
from oracle import oracle as O

pytestmark = pytest.mark.gpu

INT64_MIN = -(1 << 63)
INT64_MAX = (1 << 63) - 1
RTOL = {torch.float32: 1e-5, torch.bfloat16: 1e-2}


def announce(*parts):
    print("CASE", *parts, flush=True)
    sys.stdout.flush()


def assert_close(got, ref, rtol, atol, scale=None):
    """|got - ref| <= atol + rtol * max(|ref|, scale).

    For a sum, ``scale`` is the same sum over |terms|: fp32 summation error is
    bounded relative to it, not to a result that cancels towards zero.
    """

    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    err = np.abs(got - ref)
    mag = np.abs(ref) if scale is None else np.maximum(np.abs(ref), np.asarray(scale, dtype=np.float64))
    bound = atol + rtol * mag
    bad = err > bound
    assert not bad.any(), f"{int(bad.sum())} mismatches, worst {float((err - bound).max())}"


def to_np(t):
    if t.dtype == torch.bfloat16:
        return t.float().cpu().numpy()
    return t.cpu().numpy()


# ------------------------------------------------------------- bucketing --


def test_bucketize_pre_hashed_bit_exact(device):
    rng = np.random.default_rng(10)
    for n in (1, 7, 4096, 100_003):
        for buckets in (1, 8, 1 << 20, 1 << 40):
            announce("bucketize_pre_hashed", n, buckets)
            raw = rng.integers(INT64_MIN, INT64_MAX, size=n, dtype=np.int64, endpoint=True)
            raw[: min(n, 4)] = [INT64_MIN, INT64_MAX, 0, -1][: min(n, 4)]
            valid = (rng.random(n) > 0.1).astype(np.uint8)
            ref, zeros = O.bucketize_pre_hashed(raw, buckets, valid)
            err = torch.zeros(1, dtype=torch.int32, device=device)
            got = ops.bucketize(torch.from_numpy(raw).to(device), buckets, valid=torch.from_numpy(valid).to(device),
                                error_count=err)
            assert np.array_equal(got.cpu().numpy(), ref)
            assert int(err.item()) == zeros


def test_bucketize_mod_bit_exact(device):
    rng = np.random.default_rng(11)
    for n in (1, 5000, 65_537):
        # divisors m = rows - 1 from 1 to 2^62 (the multiply-high reduction)
        for rows in (2, 3, 6, 1_000_000, 999_999_937, (1 << 31) + 12, (1 << 40) + 2, (1 << 62) + 1):
            announce("bucketize_mod", n, rows)
            raw = rng.integers(INT64_MIN, INT64_MAX, size=n, dtype=np.int64, endpoint=True)
            raw[: min(n, 3)] = [INT64_MIN, INT64_MAX, 0][: min(n, 3)]
            got = ops.bucketize(torch.from_numpy(raw).to(device), rows, mode="mod", validate_nonzero=False)
            assert np.array_equal(got.cpu().numpy(), O.bucketize_mod(raw, rows))


def test_lengths_to_offsets_bit_exact(device):
    rng = np.random.default_rng(12)
    # up to 1024 tiles of 2048 the final kernel adds up its prefix itself;
    # 2.5 M lengths (1221 tiles) take the three-launch scan
    for n in (0, 1, 5, 2048, 2049, 100_003, 1_638_400, 2_500_000):
        announce("lengths_to_offsets", n)
        lengths = rng.integers(0, 33, size=n).astype(np.int64)
        got = ops.lengths_to_offsets(torch.from_numpy(lengths).to(device))
        assert np.array_equal(got.cpu().numpy(), O.offsets_of(lengths))


# ----------------------------------------------------------------- sort --


@pytest.mark.parametrize("bits", [1, 7, 8, 13, 24, 25, 27, 30, 31, 32])
def test_radix_sort_is_stable_and_exact(device, bits):
    """Every key width takes 8-bit passes; tiles hold 256 threads x 4, 8 or 16
    keys (16 from about 2.1 M keys, so at least 512 tiles), and the sizes
    straddle whole tiles and partial last tiles of each."""

    rng = np.random.default_rng(13 + bits)
    lib = _lib.lib()
    big = (2_000_003, 4_500_001) if bits in (24, 31) else (20_000,)
    for n in (1, 100, 1024, 1025, 4096, 4097, 8193, 16384, 16385, 300_001) + big:
        announce("sort_pairs", n, bits)
        hi = (1 << bits) - 1
        keys = rng.integers(0, hi, size=n, dtype=np.uint64, endpoint=True)
        keys[: n // 3] = keys[: n // 3] % 17  # many duplicates
        keys = keys.astype(np.uint32)
        k = torch.from_numpy(keys.view(np.int32)).to(device)
        v = torch.arange(n, dtype=torch.int32, device=device)
        k2 = torch.empty_like(k)
        v2 = torch.empty_like(v)
        ws = torch.empty(lib.mdl_sort_workspace_bytes(n), dtype=torch.uint8, device=device)
        in_alt = _lib.ctypes.c_int32(0)
        rc = lib.mdl_sort_pairs(k.data_ptr(), v.data_ptr(), k2.data_ptr(), v2.data_ptr(), n, bits, ws.data_ptr(),
                                ws.numel(), _lib.ctypes.addressof(in_alt), torch.cuda.current_stream().cuda_stream)
        _lib.check(rc, "mdl_sort_pairs")
        ks, vs = (k2, v2) if in_alt.value else (k, v)
        order = np.argsort(keys, kind="stable")
        assert np.array_equal(ks.cpu().numpy().view(np.uint32), keys[order])
        assert np.array_equal(vs.cpu().numpy(), order.astype(np.int32))


def test_unique_matches_torch_unique(device):
    rng = np.random.default_rng(14)
    for n in (1, 1000, 250_000):
        announce("unique", n)
        ids = (rng.zipf(1.1, size=n) % 1_000_003).astype(np.int64)
        u, inv, cnt = ops.unique(torch.from_numpy(ids).to(device))
        ru, rinv, rcnt = O.unique(ids)
        assert np.array_equal(u.cpu().numpy(), ru)
        assert np.array_equal(inv.cpu().numpy(), rinv)
        assert np.array_equal(cnt.cpu().numpy(), rcnt)


# -------------------------------------------------------------- forward --


def _table(rng, rows, dim, dtype, device):
    w = torch.from_numpy(rng.standard_normal((rows, dim)).astype(np.float32)).to(dtype)
    w[0] = 0
    return w.to(device)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("dim", [1, 3, 4, 8, 16, 24, 64, 128, 256, 300])
def test_gather_is_exact_copy(device, dtype, dim):
    rng = np.random.default_rng(dim)
    announce("gather", dtype, dim)
    w = _table(rng, 1000, dim, dtype, device)
    ids = torch.from_numpy(rng.integers(0, 1000, size=(37, 5))).to(device)
    plan = ops.GroupPlan()
    plan.add_feature(w, pooling="none")
    res = ops.grouped_forward(plan, [ids], [None], with_backward=False)
    out = res.outputs[0]
    assert out.shape == (37, 5, dim)
    assert torch.equal(out, w[ids])
    assert int(res.error_count.item()) == 0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("mode", ["sum", "mean"])
@pytest.mark.parametrize("policy", ["exclude", "include_as_padding"])
@pytest.mark.parametrize("dim", [4, 16, 24, 32, 64, 128, 300])
def test_pooled_forward_matches_oracle(device, dtype, mode, policy, dim):
    rng = np.random.default_rng(dim * 7 + len(mode) + len(policy))
    announce("pooled_forward", dtype, mode, policy, dim)
    rows = 5000
    w = _table(rng, rows, dim, dtype, device)
    B = 700
    lengths = rng.integers(0, 33, size=B)
    lengths[::50] = 0
    lengths[7] = 2000  # one very long bag spans many passes
    ids = rng.integers(0, rows, size=int(lengths.sum()))
    ids[::9] = 0
    plan = ops.GroupPlan()
    plan.add_feature(w, pooling=mode, null_policy=policy)
    res = ops.grouped_forward(plan, [torch.from_numpy(ids).to(device)], [torch.from_numpy(lengths).to(device)],
                              with_backward=False)
    ref, _ = O.pool(to_np(w), ids, lengths, mode, policy)
    scale, _ = O.pool(np.abs(to_np(w)), ids, lengths, mode, policy)
    assert_close(to_np(res.outputs[0]), ref, RTOL[dtype], 1e-6 if dtype == torch.float32 else 1e-2, scale)


def test_grouped_mixed_features_one_launch(device):
    """Pooled and unpooled features of several dims and two aliased tables."""

    rng = np.random.default_rng(21)
    announce("grouped_mixed")
    tabs = [_table(rng, r, d, torch.float32, device) for r, d in ((300, 16), (5000, 64), (77, 128), (1000, 32))]
    B = 257
    plan = ops.GroupPlan()
    spec = [(0, "mean", "exclude"), (1, "sum", "include_as_padding"), (2, "none", "exclude"),
            (1, "mean", "include_as_padding"), (3, "none", "exclude"), (0, "sum", "exclude")]
    ids, lens, refs = [], [], []
    for t, mode, pol in spec:
        plan.add_feature(tabs[t], pooling=mode, null_policy=pol)
        rows = tabs[t].shape[0]
        if mode == "none":
            x = rng.integers(0, rows, size=B)
            ids.append(torch.from_numpy(x).to(device))
            lens.append(None)
            refs.append(O.gather(to_np(tabs[t]), x))
        else:
            ln = rng.integers(0, 20, size=B)
            x = rng.integers(0, rows, size=int(ln.sum()))
            ids.append(torch.from_numpy(x).to(device))
            lens.append(torch.from_numpy(ln).to(device))
            refs.append(O.pool(to_np(tabs[t]), x, ln, mode, pol)[0])
    assert len(plan.tables) == 4
    res = ops.grouped_forward(plan, ids, lens, with_backward=False)
    for out, ref in zip(res.outputs, refs):
        assert_close(to_np(out), ref, 1e-5, 1e-6)


@pytest.mark.parametrize("order", ["oldest_to_newest", "newest_to_oldest"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_sequence_forward_matches_oracle(device, order, dtype):
    rng = np.random.default_rng(22)
    announce("sequence_forward", order, dtype)
    w = _table(rng, 3000, 64, dtype, device)
    B, L = 33, 200
    lengths = rng.integers(0, L + 1, size=B)
    lengths[0] = L
    ids = np.zeros((B, L), dtype=np.int64)
    for b in range(B):
        ids[b, : lengths[b]] = rng.integers(1, 3000, size=lengths[b])
    for out_len in (L, 150, 256):
        out, mask = ops.sequence_forward(w, torch.from_numpy(ids).to(device), torch.from_numpy(lengths).to(device),
                                         out_len=out_len, order=order)
        ref, rmask = O.sequence_gather(to_np(w), ids, lengths, out_len, order)
        assert np.array_equal(mask.cpu().numpy(), rmask)
        assert np.array_equal(to_np(out), ref.astype(np.float32))


@pytest.mark.parametrize("dim,dtype,out_dtype", [
    (3, torch.float32, torch.float32),      # scalar lanes (12-byte rows)
    (24, torch.float32, torch.float32),     # 8 per lane, last lane of 4 outside the row
    (128, torch.float32, torch.float32),
    (12, torch.bfloat16, torch.bfloat16),   # 24-byte rows: scalar lanes
    (40, torch.bfloat16, torch.float32),
])
@pytest.mark.parametrize("order", ["oldest_to_newest", "newest_to_oldest"])
def test_sequence_forward_widths_and_invalid_ids(device, dim, dtype, out_dtype, order):
    """Every lane-width variant of the window gather, windows shorter than
    the input rows, empty rows, and ids outside the table: those read as
    zero rows (still valid positions) and are counted once each."""
    rng = np.random.default_rng(31)
    announce("sequence_widths", dim, dtype, out_dtype, order)
    rows = 500
    w = _table(rng, rows, dim, dtype, device)
    B, L, out_len = 7, 90, 64
    lengths = rng.integers(0, L + 1, size=B)
    lengths[0], lengths[1], lengths[2] = L, 0, 10
    ids = np.zeros((B, L), dtype=np.int64)
    for b in range(B):
        ids[b, : lengths[b]] = rng.integers(1, rows, size=lengths[b])
    ids[0, 5], ids[0, 6], ids[2, 0] = rows, -3, 10**9
    ids[3, L - 1] = 10**9 if lengths[3] < L else ids[3, L - 1]  # past the row's length: not looked up
    # a row longer than the window contributes its first out_len ids (either
    # order), so all three planted ids are looked up
    err = torch.zeros(1, dtype=torch.int32, device=device)
    out, mask = ops.sequence_forward(w, torch.from_numpy(ids).to(device), torch.from_numpy(lengths).to(device),
                                     out_len=out_len, order=order, out_dtype=out_dtype, error_count=err)
    safe = np.where((ids >= 0) & (ids < rows), ids, 0)  # row 0 is zero
    ref, rmask = O.sequence_gather(to_np(w), safe, lengths, out_len, order)
    assert out.dtype == out_dtype
    assert np.array_equal(mask.cpu().numpy(), rmask)
    assert np.array_equal(to_np(out), ref.astype(np.float32))
    assert int(err.item()) == 3


def test_invalid_ids_are_counted_not_read(device):
    rng = np.random.default_rng(23)
    announce("invalid_ids")
    w = _table(rng, 100, 16, torch.float32, device)
    ids = torch.tensor([1, 2, 100, -1, 5], device=device)
    plan = ops.GroupPlan()
    plan.add_feature(w, pooling="none")
    res = ops.grouped_forward(plan, [ids], [None], with_backward=False)
    assert int(res.error_count.item()) == 2
    out = res.outputs[0]
    assert torch.equal(out[[0, 1, 4]], w[[1, 2, 5]])
    assert out[2].abs().sum() == 0 and out[3].abs().sum() == 0
    # lengths that overrun the ids are clamped and counted
    plan = ops.GroupPlan()
    plan.add_feature(w, pooling="sum")
    res = ops.grouped_forward(plan, [torch.tensor([1, 2, 3], device=device)],
                              [torch.tensor([2, 5], device=device)], with_backward=False)
    assert int(res.error_count.item()) > 0
    assert_close(to_np(res.outputs[0][0]), to_np(w[1] + w[2]), 1e-6, 1e-6)


def test_pooled_bad_lengths_and_ids_stay_in_bounds(device):
    """A negative length (decreasing offsets) and an id outside the table in
    a bag: both are counted, nothing is read out of bounds, the other bags
    pool as usual, and a bad id weighs 0 in a mean."""
    rng = np.random.default_rng(24)
    announce("pooled_bad_lengths")
    w = _table(rng, 100, 16, torch.float32, device)
    plan = ops.GroupPlan()
    plan.add_feature(w, pooling="sum")
    ids = torch.tensor([1, 2, 3, 4, 5, 6], device=device)
    res = ops.grouped_forward(plan, [ids], [torch.tensor([2, -1, 3, 2], device=device)], with_backward=False)
    assert int(res.error_count.item()) >= 1
    out = to_np(res.outputs[0])
    assert np.isfinite(out).all()
    assert_close(out[0], to_np(w[1] + w[2]), 1e-6, 1e-6)
    # offsets 0, 2, 1, 4, 6 are made non-decreasing (0, 2, 2, 4, 6): bag 1 is empty
    assert np.abs(out[1]).sum() == 0
    assert_close(out[3], to_np(w[5] + w[6]), 1e-6, 1e-6)
    plan = ops.GroupPlan()
    plan.add_feature(w, pooling="mean", null_policy="exclude")
    res = ops.grouped_forward(plan, [torch.tensor([1, 200, 3, 0, 7], device=device)],
                              [torch.tensor([3, 2], device=device)], with_backward=False)
    assert int(res.error_count.item()) == 1
    out = to_np(res.outputs[0])
    assert_close(out[0], to_np((w[1] + w[3]) / 2), 1e-6, 1e-6)  # the bad id weighs 0
    assert_close(out[1], to_np(w[7]), 1e-6, 1e-6)  # the null (0) is excluded from the mean


# -------------------------------------------------------------- backward --


def _random_group(rng, device, dtype=torch.float32, hot=False, B=300):
    dims = [16, 64, 32, 128, 24]
    rows = [50, 4000, 100_000, 700, 1000]
    tabs = [_table(rng, r, d, dtype, device) for r, d in zip(rows, dims)]
    spec = [(0, "mean", "exclude"), (1, "sum", "include_as_padding"), (2, "none", "exclude"),
            (1, "mean", "exclude"), (3, "none", "exclude"), (4, "mean", "include_as_padding")]
    plan = ops.GroupPlan()
    states = [torch.from_numpy(rng.random(r).astype(np.float32)).to(device) for r in rows]
    ids, lens, meta = [], [], []
    for t, mode, pol in spec:
        plan.add_feature(tabs[t], pooling=mode, null_policy=pol, state=states[t])
        r = rows[t]
        if mode == "none":
            x = rng.integers(0, r, size=B)
            ln = None
        else:
            ln = rng.integers(0, 40, size=B)
            x = (rng.zipf(1.2, size=int(ln.sum())) % r) if hot else rng.integers(0, r, size=int(ln.sum()))
        if hot:
            x[: len(x) // 2] = 3  # one row with thousands of entries spans many chunks
        x[::11] = 0
        ids.append(torch.from_numpy(np.asarray(x, dtype=np.int64)).to(device))
        lens.append(None if ln is None else torch.from_numpy(ln).to(device))
        meta.append((t, mode, pol, np.asarray(x), ln))
    return plan, tabs, states, ids, lens, meta, dims


@pytest.mark.parametrize("hot", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_backward_coalesce_matches_oracle(device, hot, dtype):
    rng = np.random.default_rng(30 + hot)
    announce("backward_coalesce", hot, dtype)
    plan, tabs, states, ids, lens, meta, dims = _random_group(rng, device, dtype, hot)
    res = ops.grouped_forward(plan, ids, lens, with_backward=True)
    grads = [torch.from_numpy(rng.standard_normal(tuple(o.shape)).astype(np.float32)).to(dtype).to(device)
             for o in res.outputs]
    out = ops.backward_coalesce(res, grads)
    for t in range(len(tabs)):
        rs, vs = [], []
        for f, (tt, mode, pol, x, ln) in enumerate(meta):
            if tt != t:
                continue
            g = to_np(grads[f]).reshape(-1, dims[t])
            r, v = O.per_id_grads(x, ln, g, mode, pol)
            rs.append(r)
            vs.append(v)
        rr, vv = O.coalesce(np.concatenate(rs), np.concatenate(vs))
        _, vabs = O.coalesce(np.concatenate(rs), np.abs(np.concatenate(vs)))
        rows, vals = out[t]
        assert np.array_equal(rows.cpu().numpy(), rr), f"table {t} rows"
        assert_close(to_np(vals), vv, RTOL[dtype], 1e-5 if dtype == torch.float32 else 1e-2, vabs)


@pytest.mark.parametrize("hot", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_fused_backward_adagrad_matches_oracle(device, hot, dtype):
    rng = np.random.default_rng(40 + hot)
    announce("fused_backward_adagrad", hot, dtype)
    plan, tabs, states, ids, lens, meta, dims = _random_group(rng, device, dtype, hot)
    w0 = [to_np(t).copy() for t in tabs]
    a0 = [s.cpu().numpy().copy() for s in states]
    res = ops.grouped_forward(plan, ids, lens, with_backward=True)
    grads = [torch.from_numpy(rng.standard_normal(tuple(o.shape)).astype(np.float32)).to(dtype).to(device)
             for o in res.outputs]
    lr, eps = 0.01, 1e-8
    ops.backward_adagrad(res, grads, lr=lr, eps=eps)
    for t in range(len(tabs)):
        rs, vs = [], []
        for f, (tt, mode, pol, x, ln) in enumerate(meta):
            if tt != t:
                continue
            r, v = O.per_id_grads(x, ln, to_np(grads[f]).reshape(-1, dims[t]), mode, pol)
            rs.append(r)
            vs.append(v)
        rr, vv = O.coalesce(np.concatenate(rs), np.concatenate(vs))
        wexp, aexp = O.rowwise_adagrad(w0[t], a0[t], rr, vv, lr, eps, is_bf16=dtype == torch.bfloat16)
        assert_close(states[t].cpu().numpy(), aexp, 1e-5, 1e-7)
        assert_close(to_np(tabs[t]), wexp, RTOL[dtype], 1e-6 if dtype == torch.float32 else 1e-2)
        untouched = np.setdiff1d(np.arange(w0[t].shape[0]), rr)
        assert np.array_equal(to_np(tabs[t])[untouched], w0[t][untouched])


@pytest.mark.parametrize("scale", [1.0, 0.52])
def test_fused_backward_large_call_matches_oracle(device, scale):
    """Calls of 1.9 M and 1.0 M ids: slots walk 48 and 30 entries per chunk
    (n / 32768, from 16 for the small calls of the other tests to 48)."""

    rng = np.random.default_rng(45)
    announce("fused_backward_large", scale)
    rows, dims = [200_000, 50_000], [16, 64]
    tabs = [_table(rng, r, d, torch.float32, device) for r, d in zip(rows, dims)]
    states = [torch.from_numpy(rng.random(r).astype(np.float32)).to(device) for r in rows]
    plan = ops.GroupPlan()
    ids, lens, meta = [], [], []
    for t, mode, B in ((0, "mean", int(60_000 * scale)), (1, "sum", int(35_000 * scale))):
        plan.add_feature(tabs[t], pooling=mode, null_policy="exclude", state=states[t])
        ln = rng.integers(0, 41, size=B)
        x = rng.zipf(1.1, size=int(ln.sum())) % rows[t]
        ids.append(torch.from_numpy(x.astype(np.int64)).to(device))
        lens.append(torch.from_numpy(ln).to(device))
        meta.append((t, mode, x, ln))
    n = sum(m[2].size for m in meta)
    assert (n > 48 * 32768) if scale == 1.0 else (20 * 32768 < n < 40 * 32768)
    w0 = [to_np(t).copy() for t in tabs]
    a0 = [s.cpu().numpy().copy() for s in states]
    res = ops.grouped_forward(plan, ids, lens, with_backward=True)
    grads = [torch.from_numpy(rng.standard_normal(tuple(o.shape)).astype(np.float32)).to(device)
             for o in res.outputs]
    lr, eps = 0.01, 1e-8
    ops.backward_adagrad(res, grads, lr=lr, eps=eps)
    for f, (t, mode, x, ln) in enumerate(meta):
        r, v = O.per_id_grads(x, ln, to_np(grads[f]).reshape(-1, dims[t]), mode, "exclude")
        rr, vv = O.coalesce(r, v)
        wexp, aexp = O.rowwise_adagrad(w0[t], a0[t], rr, vv, lr, eps)
        assert_close(states[t].cpu().numpy(), aexp, 1e-5, 1e-7)
        assert_close(to_np(tabs[t]), wexp, 1e-5, 1e-6)


def test_fused_backward_is_deterministic(device):
    announce("determinism")
    results = []
    for _ in range(2):
        rng = np.random.default_rng(50)
        plan, tabs, states, ids, lens, meta, dims = _random_group(rng, device, torch.float32, True)
        res = ops.grouped_forward(plan, ids, lens, with_backward=True)
        grads = [torch.from_numpy(rng.standard_normal(tuple(o.shape)).astype(np.float32)).to(device)
                 for o in res.outputs]
        ops.backward_adagrad(res, grads, lr=0.01, eps=1e-8)
        results.append([t.cpu().clone() for t in tabs] + [s.cpu().clone() for s in states])
    for a, b in zip(*results):
        assert torch.equal(a, b)


@pytest.mark.parametrize("big_rows,dtype,dim", [((1 << 25) + 3, torch.float32, 8),
                                                ((1 << 30) + 5, torch.bfloat16, 2)])
def test_clipped_step_with_wide_keys(device, big_rows, dtype, dim):
    """The clipped step sorts (mdl_backward_sort), then reduces the sorted
    pairs twice (mdl_backward_sumsq, mdl_backward_apply), which must find them
    where the sort's pass count left them; 26- and 31-bit keys (four passes)
    and the hot last row of a table of 2^30 rows."""

    rng = np.random.default_rng(71)
    announce("clipped_wide_keys", big_rows, dtype, dim)
    big = torch.zeros((big_rows, dim), dtype=dtype, device=device)
    big_state = torch.zeros(big_rows, dtype=torch.float32, device=device)
    small = _table(rng, 3000, 16, dtype, device)
    small_state = torch.from_numpy(rng.random(3000).astype(np.float32)).to(device)
    tabs, states, dims = [big, small], [big_state, small_state], [dim, 16]
    plan = ops.GroupPlan()
    ids, lens, meta = [], [], []
    for t, pool in ((0, "mean"), (1, "sum"), (0, "none")):
        plan.add_feature(tabs[t], pooling=pool, null_policy="exclude", state=states[t])
        rows = tabs[t].shape[0]
        ln = None if pool == "none" else rng.integers(0, 24, size=1500)
        n = 1500 if ln is None else int(ln.sum())
        x = rng.integers(0, rows, size=n)
        x[rng.random(n) < 0.3] = rows - 1  # the table's last row: the widest keys
        x[::13] = 0
        ids.append(torch.from_numpy(x.astype(np.int64)).to(device))
        lens.append(None if ln is None else torch.from_numpy(ln).to(device))
        meta.append((t, pool, x, ln))
    assert plan.key_bits == int(big_rows + 3000).bit_length() and plan.key_bits > 24
    touched = np.unique(np.concatenate([m[2] for m in meta if m[0] == 0]))
    tidx = torch.from_numpy(touched).to(device)
    big[tidx] = torch.from_numpy(rng.standard_normal((touched.size, dim)).astype(np.float32)).to(dtype).to(device)
    big_state[tidx] = torch.from_numpy(rng.random(touched.size).astype(np.float32)).to(device)
    w0 = [to_np(big[tidx]).copy(), to_np(small).copy()]
    a0 = [big_state[tidx].cpu().numpy().copy(), small_state.cpu().numpy().copy()]
    res = ops.grouped_forward(plan, ids, lens, with_backward=True)
    grads = [torch.from_numpy(rng.standard_normal(tuple(o.shape)).astype(np.float32)).to(dtype).to(device)
             for o in res.outputs]
    rows_vals = []
    for t in range(2):
        rs, vs = [], []
        for f, (tt, pool, x, ln) in enumerate(meta):
            if tt == t:
                r, v = O.per_id_grads(x, ln, to_np(grads[f]).reshape(-1, dims[t]), pool, "exclude")
                rs.append(r)
                vs.append(v)
        rows_vals.append(O.coalesce(np.concatenate(rs), np.concatenate(vs)))
    scaled, total, _ = O.clip_grad_norm([v for _, v in rows_vals], 1.0)
    lr, eps = 0.01, 1e-8
    norm = ops.backward_adagrad(res, grads, lr=lr, eps=eps, clip_norm=1.0)
    assert abs(float(norm.item()) - total) <= 1e-4 * total
    tol = (1e-5, 1e-6) if dtype == torch.float32 else (1e-2, 1e-2)
    # table 0: compare its touched rows (the oracle runs on them compacted)
    rr = rows_vals[0][0]
    pos = np.searchsorted(touched, rr)
    wexp, aexp = O.rowwise_adagrad(w0[0][pos], a0[0][pos], np.arange(rr.size), scaled[0], lr, eps,
                                   is_bf16=dtype == torch.bfloat16)
    rr_dev = torch.from_numpy(rr).to(device)
    assert_close(to_np(big[rr_dev]), wexp, *tol)
    assert_close(big_state[rr_dev].cpu().numpy(), aexp, 1e-5, 1e-7)
    untouched = np.setdiff1d(touched, rr)
    assert np.array_equal(to_np(big[torch.from_numpy(untouched).to(device)]), w0[0][np.searchsorted(touched, untouched)])
    wexp, aexp = O.rowwise_adagrad(w0[1], a0[1], rows_vals[1][0], scaled[1], lr, eps, is_bf16=dtype == torch.bfloat16)
    assert_close(to_np(small), wexp, *tol)
    assert_close(small_state.cpu().numpy(), aexp, 1e-5, 1e-7)


@pytest.mark.parametrize("mode", ["coalesce", "adagrad", "clipped"])
def test_hot_row_spanning_hundreds_of_chunks(device, mode):
    """A Zipf head row whose run covers several hundred chunks (the fix-up
    searches back over such chunks 64 at a time); a second hot row follows it
    in the same table, and a dim-16 table has a run of ~150 chunks."""

    rng = np.random.default_rng(60)
    announce("hot_row_chunks", mode)
    dims, rows = [128, 16], [5000, 3000]
    tabs = [_table(rng, r, d, torch.float32, device) for r, d in zip(rows, dims)]
    states = [torch.from_numpy(rng.random(r).astype(np.float32)).to(device) for r in rows]
    plan = ops.GroupPlan()
    ids, lens, meta = [], [], []
    for t, pool in ((0, "mean"), (1, "sum"), (0, "sum")):
        plan.add_feature(tabs[t], pooling=pool, null_policy="exclude", state=states[t])
        ln = rng.integers(20, 80, size=2048)
        x = rng.integers(0, rows[t], size=int(ln.sum()))
        x[rng.random(x.size) < 0.8] = 7
        x[rng.random(x.size) < 0.1] = 9
        ids.append(torch.from_numpy(x.astype(np.int64)).to(device))
        lens.append(torch.from_numpy(ln).to(device))
        meta.append((t, pool, x, ln))
    w0 = [to_np(t).copy() for t in tabs]
    a0 = [s.cpu().numpy().copy() for s in states]
    res = ops.grouped_forward(plan, ids, lens, with_backward=True)
    grads = [torch.from_numpy(rng.standard_normal(tuple(o.shape)).astype(np.float32)).to(device)
             for o in res.outputs]
    expect = []
    for t in range(len(tabs)):
        rs, vs = [], []
        for f, (tt, pool, x, ln) in enumerate(meta):
            if tt == t:
                r, v = O.per_id_grads(x, ln, to_np(grads[f]).reshape(-1, dims[t]), pool, "exclude")
                rs.append(r)
                vs.append(v)
        expect.append((O.coalesce(np.concatenate(rs), np.concatenate(vs)),
                       O.coalesce(np.concatenate(rs), np.abs(np.concatenate(vs)))[1]))
    assert np.count_nonzero(expect[0][0][0] == 7) == 1
    if mode == "coalesce":
        out = ops.backward_coalesce(res, grads)
        for t, ((rr, vv), vabs) in enumerate(expect):
            got_rows, got_vals = out[t]
            assert np.array_equal(got_rows.cpu().numpy(), rr), f"table {t} rows"
            assert_close(to_np(got_vals), vv, 1e-5, 1e-5, vabs)
        return
    lr, eps = 0.01, 1e-8
    vals = [vv for (_, vv), _ in expect]
    if mode == "clipped":
        vals, total, _ = O.clip_grad_norm(vals, 1.0)
        norm = ops.backward_adagrad(res, grads, lr=lr, eps=eps, clip_norm=1.0)
        assert abs(float(norm.item()) - total) <= 1e-5 * total
    else:
        ops.backward_adagrad(res, grads, lr=lr, eps=eps)
    for t, ((rr, _), _) in enumerate(expect):
        wexp, aexp = O.rowwise_adagrad(w0[t], a0[t], rr, vals[t], lr, eps)
        assert_close(states[t].cpu().numpy(), aexp, 1e-5, 1e-7)
        assert_close(to_np(tabs[t]), wexp, 1e-5, 1e-6)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("dim", [2, 16, 24, 48, 66, 100, 128, 256, 300, 384, 520])
def test_rowwise_adagrad_matches_oracle(device, dtype, dim):
    """Any dim, like the reference kernel (BLOCK = next_pow2(dim)): rows
    wider than 64 lanes cover (fp32 300/384/520, unaligned 66/100) take the
    column-block walk."""
    rng = np.random.default_rng(60 + dim)
    announce("rowwise_adagrad", dtype, dim)
    rows = 3000
    w = _table(rng, rows, dim, dtype, device)
    acc = torch.from_numpy(rng.random(rows).astype(np.float32)).to(device)
    touched = rng.choice(rows, size=900, replace=False)
    vals = rng.standard_normal((900, dim)).astype(np.float32)
    vt = torch.from_numpy(vals).to(dtype).to(device)
    wexp, aexp = O.rowwise_adagrad(to_np(w), acc.cpu().numpy(), touched, to_np(vt), 0.05, 1e-8,
                                   is_bf16=dtype == torch.bfloat16)
    ops.rowwise_adagrad_(w, acc, torch.from_numpy(touched).to(device), vt, lr=0.05, eps=1e-8)
    assert_close(acc.cpu().numpy(), aexp, 1e-5, 1e-7)
    assert_close(to_np(w), wexp, RTOL[dtype], 1e-6 if dtype == torch.float32 else 1e-2)


def test_coalesce_rows_matches_torch(device):
    rng = np.random.default_rng(70)
    announce("coalesce_rows")
    n, dim, rows = 50_000, 32, 10_000
    idx = (rng.zipf(1.1, size=n) % rows).astype(np.int64)
    vals = rng.standard_normal((n, dim)).astype(np.float32)
    r, v = ops.coalesce_rows(torch.from_numpy(idx).to(device), torch.from_numpy(vals).to(device), rows)
    rr, vv = O.coalesce(idx, vals.astype(np.float64))
    _, vabs = O.coalesce(idx, np.abs(vals.astype(np.float64)))
    assert np.array_equal(r.cpu().numpy(), rr)
    assert_close(v.cpu().numpy(), vv, 1e-5, 1e-6, vabs)


# Rows wider than 64 lanes cover (fp32 300 with 4 per lane, 600 and 1030
# unaligned, 66 unaligned; bf16 100 unaligned, 600 with 8 per lane): one wave
# per run walks them in column blocks.
WIDE = [(66, torch.float32), (300, torch.float32), (600, torch.float32), (1030, torch.float32),
        (100, torch.bfloat16), (600, torch.bfloat16)]


@pytest.mark.parametrize("dim,dtype", WIDE)
def test_coalesce_rows_wide_rows_match_oracle(device, dim, dtype):
    announce("coalesce_rows_wide", dim, dtype)
    rng = np.random.default_rng(72 + dim)
    n, rows = 6000, 900
    idx = (rng.zipf(1.2, size=n) % rows).astype(np.int64)
    idx[: n // 3] = 5  # a run over many chunks (the fix-up)
    vals = torch.from_numpy(rng.standard_normal((n, dim)).astype(np.float32)).to(dtype)
    r, v = ops.coalesce_rows(torch.from_numpy(idx).to(device), vals.to(device), rows)
    rr, vv = O.coalesce(idx, vals.float().numpy().astype(np.float64))
    _, vabs = O.coalesce(idx, np.abs(vals.float().numpy().astype(np.float64)))
    assert np.array_equal(r.cpu().numpy(), rr)
    assert_close(to_np(v), vv, RTOL[dtype], 1e-5 if dtype == torch.float32 else 1e-2, vabs)


@pytest.mark.parametrize("hot", [False, True])
@pytest.mark.parametrize("dim,dtype", WIDE)
def test_fused_backward_wide_rows_match_oracle(device, dim, dtype, hot):
    """Pooled (mean, sum) and unpooled features on a wide table beside a
    narrow one, through the fused reduce + row-wise Adagrad, the coalesce and
    the clip's squared norm."""

    announce("fused_backward_wide", dim, dtype, hot)
    rng = np.random.default_rng(80 + dim + hot)
    rows, dims = [700, 3000], [dim, 32]
    B = 200
    tabs = [_table(rng, r, d, dtype, device) for r, d in zip(rows, dims)]
    states = [torch.from_numpy(rng.random(r).astype(np.float32)).to(device) for r in rows]
    plan = ops.GroupPlan()
    ids, lens, meta = [], [], []
    for t, mode in ((0, "mean"), (1, "sum"), (0, "none"), (0, "sum")):
        plan.add_feature(tabs[t], pooling=mode, null_policy="exclude", state=states[t])
        ln = None if mode == "none" else rng.integers(0, 30, size=B)
        m = B if ln is None else int(ln.sum())
        x = (rng.zipf(1.2, size=m) % rows[t]) if hot else rng.integers(0, rows[t], size=m)
        if hot:
            x[: m // 2] = 7
        x[::13] = 0
        ids.append(torch.from_numpy(np.asarray(x, dtype=np.int64)).to(device))
        lens.append(None if ln is None else torch.from_numpy(ln).to(device))
        meta.append((t, mode, np.asarray(x), ln))
    res = ops.grouped_forward(plan, ids, lens, with_backward=True)
    grads = [torch.from_numpy(rng.standard_normal(tuple(o.shape)).astype(np.float32)).to(dtype).to(device)
             for o in res.outputs]
    expect, vabs = [], []
    for t in range(2):
        rs, vs = [], []
        for f, (tt, mode, x, ln) in enumerate(meta):
            if tt == t:
                r, v = O.per_id_grads(x, ln, to_np(grads[f]).reshape(-1, dims[t]), mode, "exclude")
                rs.append(r)
                vs.append(v)
        expect.append(O.coalesce(np.concatenate(rs), np.concatenate(vs)))
        vabs.append(O.coalesce(np.concatenate(rs), np.abs(np.concatenate(vs)))[1])
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    out = ops.backward_coalesce(res, grads)
    for t in range(2):
        rows_t, vals_t = out[t]
        assert np.array_equal(rows_t.cpu().numpy(), expect[t][0]), t
        assert_close(to_np(vals_t), expect[t][1], RTOL[dtype], tol, vabs[t])
    # The clipped update (sort, squared norm, coefficient, apply) with a bound
    # the norm stays under: the coefficient is 1 and the step the plain one.
    w0 = [to_np(t).copy() for t in tabs]
    a0 = [s.cpu().numpy().copy() for s in states]
    lr, eps = 0.01, 1e-8
    res = ops.grouped_forward(plan, ids, lens, with_backward=True)
    norm = ops.backward_adagrad(res, grads, lr=lr, eps=eps, clip_norm=1e30)
    ref = np.sqrt(sum(float((v.astype(np.float64) ** 2).sum()) for _, v in expect))
    assert abs(float(norm.item()) - ref) <= 1e-4 * ref
    for t in range(2):
        rr, vv = expect[t]
        wexp, aexp = O.rowwise_adagrad(w0[t], a0[t], rr, vv, lr, eps, is_bf16=dtype == torch.bfloat16)
        assert_close(states[t].cpu().numpy(), aexp, 1e-5, 1e-7)
        assert_close(to_np(tabs[t]), wexp, RTOL[dtype], 1e-6 if dtype == torch.float32 else 1e-2)
        untouched = np.setdiff1d(np.arange(rows[t]), rr)
        assert np.array_equal(to_np(tabs[t])[untouched], w0[t][untouched])


def _oracle_step_pooled(W, rows, dims, pools, ids, lens, grad, lr, eps, accs=None):
    """Oracle of one SparseStep over full tables (copies updated in place)."""
    B = grad.shape[0]
    cols = np.concatenate([[0], np.cumsum(dims)[:-1]])
    feats, offs, bag_off, ids_off = [], [], 0, 0
    for t, (p, x, ln) in enumerate(zip(pools, ids, lens)):
        feats.append({"table": t, "pooling": {"none": 0, "sum": 1, "mean": 2}[p], "exclude": 1, "ids_off": ids_off,
                      "bag_off": bag_off, "num_bags": 0 if ln is None else B, "out_col": int(cols[t])})
        if ln is not None:
            o = O.offsets_of(ln)
            offs.append(o)
            bag_off += len(o)
        ids_off += x.size
    tables = [{"W": w, "acc": a} for w, a in zip(W, accs)]
    out = O.sparse_step(feats, tables, np.concatenate(ids), np.concatenate(offs), sum(dims), grad, lr, eps)
    absw = [{"W": np.abs(w), "acc": np.zeros(r, np.float32)} for w, r in zip(W, rows)]
    scale = O.sparse_step(feats, absw, np.concatenate(ids), np.concatenate(offs), sum(dims), np.zeros_like(grad),
                          0.0, 1.0)
    return out, scale


def test_sparse_step_serves_batches_of_any_bag_lengths(device):
    """One SparseStep, bound to four batches whose bag lengths (and so id
    counts) differ, including one with fewer ids and one with more than the
    batch it was built from: each step matches the oracle continuing from
    the previous step's tables."""

    from mdl_amd.sparse_step import SparseStep

    rng = np.random.default_rng(84)
    B = 384
    rows = [2500, 700, 9000, 300]
    dims = [32, 16, 64, 24]
    pools = ["mean", "none", "sum", "mean"]
    W = [rng.standard_normal((r, d)).astype(np.float32) for r, d in zip(rows, dims)]
    for w in W:
        w[0] = 0
    tabs = [torch.from_numpy(w.copy()).to(device) for w in W]
    accs = [torch.zeros(r, device=device) for r in rows]
    ref_acc = [np.zeros(r, np.float32) for r in rows]
    plan = ops.GroupPlan()
    for t, p in enumerate(pools):
        plan.add_feature(tabs[t], pooling=p, null_policy="exclude", state=accs[t])
    S = sum(dims)
    cols = np.concatenate([[0], np.cumsum(dims)[:-1]])
    out = torch.empty((B, S), device=device)
    grad = torch.empty((B, S), device=device)
    views = [slice(int(c), int(c) + d) for c, d in zip(cols, dims)]

    def batch(max_len):
        ids, lens = [], []
        for t, p in enumerate(pools):
            if p == "none":
                ids.append((rng.zipf(1.2, size=B) % rows[t]).astype(np.int64))
                lens.append(None)
            else:
                ln = rng.integers(0, max_len + 1, size=B)
                ids.append((rng.zipf(1.2, size=int(ln.sum())) % rows[t]).astype(np.int64))
                lens.append(ln)
        parts = [ln if ln is not None else np.array([x.size]) for x, ln in zip(ids, lens)]
        return ids, lens, torch.from_numpy(np.concatenate(ids)).to(device), \
            torch.from_numpy(np.concatenate(parts).astype(np.int64)).to(device)

    batches = [batch(m) for m in (12, 3, 30, 12)]
    cap = max(int(b[2].numel()) for b in batches)
    ids0, lens0, p0, l0 = batches[0]
    st = SparseStep(plan, p0, l0, [x.size for x in ids0], [0 if ln is None else B for ln in lens0],
                    [out[:, v] for v in views], [grad[:, v] for v in views], capacity=cap)
    for k, (ids, lens, packed, lengths) in enumerate(batches):
        announce("sparse_step_rebind", k, int(packed.numel()))
        g = rng.standard_normal((B, S)).astype(np.float32)
        grad.copy_(torch.from_numpy(g))
        st.bind(packed, lengths)
        st.step(0.02, 1e-8)
        ref_out, scale = _oracle_step_pooled(W, rows, dims, pools, ids, lens, g.astype(np.float64), 0.02, 1e-8,
                                             ref_acc)
        assert_close(out.cpu().numpy(), ref_out, 1e-5, 1e-6, scale)
        for t in range(len(rows)):
            assert_close(accs[t].cpu().numpy(), ref_acc[t], 1e-5, 1e-6)
            assert_close(tabs[t].cpu().numpy(), W[t], 1e-5, 1e-5)
            # continue from the device's tables so tolerances do not compound
            W[t][:] = tabs[t].cpu().numpy()
            ref_acc[t][:] = accs[t].cpu().numpy()
    assert int(st.error_count.item()) == 0
    with pytest.raises(ValueError):
        st.bind(torch.zeros(cap + 1, dtype=torch.int64, device=device), batches[0][3])


def test_sparse_step_accumulates_micro_batches(device):
    """SparseStep(micro_batches=3): three micro-batches with different bag
    lengths are looked up on the same tables into their own outputs, then one
    sort + one reduce updates every row once.  Outputs match the oracle's
    lookups; tables and accumulators match one row-wise Adagrad step on the
    coalesced sum of the three micro-batches' sparse gradients, and the clip
    norm is that sum's global norm (gradient accumulation,
    src/train.py:7007-7067)."""

    from mdl_amd.sparse_step import SparseStep

    rng = np.random.default_rng(85)
    B, k, lr, eps = 256, 3, 0.03, 1e-8
    rows = [2500, 700, 9000, 300]
    dims = [32, 16, 64, 24]
    pools = ["mean", "none", "sum", "mean"]
    W = [rng.standard_normal((r, d)).astype(np.float32) for r, d in zip(rows, dims)]
    for w in W:
        w[0] = 0
    tabs = [torch.from_numpy(w.copy()).to(device) for w in W]
    accs = [torch.from_numpy(rng.random(r).astype(np.float32)).to(device) for r in rows]
    acc0 = [a.cpu().numpy() for a in accs]
    plan = ops.GroupPlan()
    for t, p in enumerate(pools):
        plan.add_feature(tabs[t], pooling=p, null_policy="exclude", state=accs[t])
    S = sum(dims)
    cols = np.concatenate([[0], np.cumsum(dims)[:-1]])
    views = [slice(int(c), int(c) + d) for c, d in zip(cols, dims)]
    outs = [torch.empty((B, S), device=device) for _ in range(k)]
    grads = [torch.empty((B, S), device=device) for _ in range(k)]

    def batch(max_len):
        ids, lens = [], []
        for t, p in enumerate(pools):
            if p == "none":
                ids.append((rng.zipf(1.2, size=B) % rows[t]).astype(np.int64))
                lens.append(None)
            else:
                ln = rng.integers(0, max_len + 1, size=B)
                ids.append((rng.zipf(1.2, size=int(ln.sum())) % rows[t]).astype(np.int64))
                lens.append(ln)
        parts = [ln if ln is not None else np.array([x.size]) for x, ln in zip(ids, lens)]
        return ids, lens, torch.from_numpy(np.concatenate(ids)).to(device), \
            torch.from_numpy(np.concatenate(parts).astype(np.int64)).to(device)

    batches = [batch(m) for m in (12, 3, 30)]
    cap = max(int(b[2].numel()) for b in batches)
    ids0, lens0, p0, l0 = batches[0]
    st = SparseStep(plan, p0, l0, [x.size for x in ids0], [0 if ln is None else B for ln in lens0],
                    [[o[:, v] for v in views] for o in outs], [[g[:, v] for v in views] for g in grads],
                    capacity=cap, micro_batches=k)
    g_host = []
    for m, (ids, lens, packed, lengths) in enumerate(batches):
        announce("sparse_step_micro_batch", m, int(packed.numel()))
        g = rng.standard_normal((B, S)).astype(np.float32)
        g_host.append(g)
        grads[m].copy_(torch.from_numpy(g))
        st.bind(packed, lengths)
        st.forward(micro_batch=m)
    st.sort()
    norm, _ = st.clip(1e9)
    st.apply(lr, eps)
    torch.cuda.synchronize()
    assert int(st.error_count.item()) == 0
    sumsq = 0.0
    for m, (ids, lens, _, _) in enumerate(batches):
        got = outs[m].cpu().numpy()
        for t, p in enumerate(pools):
            ref = O.gather(W[t], ids[t]) if p == "none" else O.pool(W[t], ids[t], lens[t], p, "exclude")[0]
            assert_close(got[:, views[t]], ref, 1e-5, 1e-6, O.pool(np.abs(W[t]), ids[t], lens[t], "sum",
                                                                   "exclude")[0] if p != "none" else None)
    for t, p in enumerate(pools):
        parts = [O.per_id_grads(b[0][t], b[1][t], g_host[m][:, views[t]].astype(np.float64), p, "exclude")
                 for m, b in enumerate(batches)]
        r, v = O.coalesce(np.concatenate([x[0] for x in parts]), np.concatenate([x[1] for x in parts]))
        sumsq += float((v * v).sum())
        w_ref, a_ref = O.rowwise_adagrad(W[t], acc0[t], r, v, lr, eps)
        assert_close(accs[t].cpu().numpy(), a_ref, 1e-5, 1e-6)
        assert_close(tabs[t].cpu().numpy(), w_ref, 1e-5, 1e-5)
    assert_close(norm.cpu().numpy(), np.array([np.sqrt(sumsq)]), 1e-5, 0)
    with pytest.raises(ValueError):
        st.forward(micro_batch=k)
    with pytest.raises(ValueError):
        st.step(lr, eps)
    st.forward(micro_batch=0)
    with pytest.raises(RuntimeError, match=r"micro-batches \[1, 2\] were not looked up"):
        st.sort()


def test_sparse_step_slot_buffer_matches_oracle(device):
    """SparseStep: pooled + unpooled features written into one [B, sum(dim)]
    slot buffer, gradients read from the same layout, fused update."""

    from mdl_amd.sparse_step import SparseStep

    announce("sparse_step")
    rng = np.random.default_rng(80)
    B = 512
    rows = [3000, 500, 20000, 64]
    dims = [32, 16, 64, 128]
    pools = ["mean", "none", "mean", "sum"]
    W = [rng.standard_normal((r, d)).astype(np.float32) for r, d in zip(rows, dims)]
    for w in W:
        w[0] = 0
    tabs = [torch.from_numpy(w.copy()).to(device) for w in W]
    accs = [torch.zeros(r, device=device) for r in rows]
    plan = ops.GroupPlan()
    for t, p in enumerate(pools):
        plan.add_feature(tabs[t], pooling=p, null_policy="exclude", state=accs[t])
    ids, lens = [], []
    for t, p in enumerate(pools):
        if p == "none":
            ids.append(rng.zipf(1.1, size=B) % rows[t])
            lens.append(None)
        else:
            ln = rng.integers(0, 25, size=B)
            ids.append(rng.zipf(1.1, size=int(ln.sum())) % rows[t])
            lens.append(ln)
    S = sum(dims)
    out = torch.empty((B, S), device=device)
    grad = torch.from_numpy(rng.standard_normal((B, S)).astype(np.float32)).to(device)
    cols = np.concatenate([[0], np.cumsum(dims)[:-1]])
    parts = [ln if ln is not None else np.array([x.size]) for x, ln in zip(ids, lens)]
    st = SparseStep(plan, torch.from_numpy(np.concatenate(ids)).to(device),
                    torch.from_numpy(np.concatenate(parts)).to(device), [x.size for x in ids],
                    [0 if ln is None else ln.size for ln in lens],
                    [out[:, c: c + d] for c, d in zip(cols, dims)], [grad[:, c: c + d] for c, d in zip(cols, dims)])
    st.step(0.02, 1e-8)
    feats = []
    offs, bag_off, ids_off = [], 0, 0
    for t, (p, x, ln) in enumerate(zip(pools, ids, lens)):
        feats.append({"table": t, "pooling": {"none": 0, "sum": 1, "mean": 2}[p], "exclude": 1, "ids_off": ids_off,
                      "bag_off": bag_off, "num_bags": 0 if ln is None else B, "out_col": int(cols[t])})
        if ln is not None:
            o = O.offsets_of(ln)
            offs.append(o)
            bag_off += len(o)
        ids_off += x.size
    tables = [{"W": w.copy(), "acc": np.zeros(r, np.float32)} for w, r in zip(W, rows)]
    ref_out = O.sparse_step(feats, tables, np.concatenate(ids), np.concatenate(offs), S,
                            grad.cpu().numpy().astype(np.float64), 0.02, 1e-8)
    absw = [{"W": np.abs(w), "acc": np.zeros(r, np.float32)} for w, r in zip(W, rows)]
    scale = O.sparse_step(feats, absw, np.concatenate(ids), np.concatenate(offs), S,
                          np.zeros((B, S)), 0.0, 1.0)
    assert_close(out.cpu().numpy(), ref_out, 1e-5, 1e-6, scale)
    for t in range(len(rows)):
        assert_close(tabs[t].cpu().numpy(), tables[t]["W"], 1e-5, 1e-6)
        assert_close(accs[t].cpu().numpy(), tables[t]["acc"], 1e-5, 1e-7)


@pytest.mark.parametrize("L_out,order,dtype", [(256, "oldest_to_newest", torch.float32),
                                               (128, "oldest_to_newest", torch.float32),
                                               (256, "newest_to_oldest", torch.float32),
                                               (128, "newest_to_oldest", torch.bfloat16)])
def test_sequence_step_matches_oracle(device, L_out, order, dtype):
    """SequenceStep sorts packed keys (only the min(len, L_in, L_out)
    positions of each row that reach the window); a window shorter than the
    input clamps the lengths, and newest-first rows reverse the positions."""
    from mdl_amd.sparse_step import SequenceStep

    announce("sequence_step", L_out, order, dtype)
    rng = np.random.default_rng(81)
    B, L = 64, 256
    rows = [4000, 9000]
    tabs = [_table(rng, r, 64, dtype, device) for r in rows]
    W = [to_np(t).copy() for t in tabs]
    accs = [torch.zeros(r, device=device) for r in rows]
    plan = ops.GroupPlan()
    for t in range(2):
        plan.add_feature(tabs[t], pooling="none", state=accs[t])
    ids, lens = [], []
    for t in range(2):
        ln = rng.integers(0, L + 1, size=B)
        m = np.zeros((B, L), dtype=np.int64)
        for b in range(B):
            m[b, : ln[b]] = rng.zipf(1.05, size=ln[b]) % rows[t]
        ids.append(m)
        lens.append(ln)
    outs = [torch.empty((B, L_out, 64), dtype=dtype, device=device) for _ in range(2)]
    masks = [torch.empty((B, L_out), dtype=torch.bool, device=device) for _ in range(2)]
    grads = [torch.from_numpy(rng.standard_normal((B, L_out, 64)).astype(np.float32)).to(dtype).to(device)
             for _ in range(2)]
    st = SequenceStep(plan, [torch.from_numpy(m).to(device) for m in ids],
                      [torch.from_numpy(ln).to(device) for ln in lens], outs, masks, grads, order=order)
    st.step(0.03, 1e-8)
    assert int(st.count.item()) == sum(int(np.minimum(ln, L_out).sum()) for ln in lens)
    bf16 = dtype == torch.bfloat16
    for t in range(2):
        ref, rmask = O.sequence_gather(W[t], ids[t], lens[t], L_out, order)
        assert np.array_equal(to_np(outs[t]), ref.astype(np.float32))
        assert np.array_equal(masks[t].cpu().numpy(), rmask)
        g = to_np(grads[t])
        r, v = [], []
        for b in range(B):
            n = int(min(lens[t][b], L_out))
            for k in range(n):
                if ids[t][b, k] != 0:
                    p = L_out - n + k if order == "oldest_to_newest" else L_out - 1 - k
                    r.append(ids[t][b, k])
                    v.append(g[b, p])
        rr, vv = O.coalesce(np.array(r), np.array(v, dtype=np.float64))
        wexp, aexp = O.rowwise_adagrad(W[t], np.zeros(rows[t], np.float32), rr, vv, 0.03, 1e-8, is_bf16=bf16)
        assert_close(to_np(tabs[t]), wexp, RTOL[dtype], 1e-2 if bf16 else 1e-6)
        assert_close(accs[t].cpu().numpy(), aexp, 1e-5, 1e-7)


# ---------------------------------------------------------------- graphs --


def _slot_step(device, seed):
    """A fixed-layout SparseStep (two tables, a mean-pooled bag feature and a
    single-valued one, outputs in one [B, sum(dim)] slot buffer)."""
    from mdl_amd.sparse_step import SparseStep

    rng = np.random.default_rng(seed)
    B = 512
    rows, dims = [3000, 20000], [32, 16]
    tabs = [_table(rng, r, d, torch.float32, device) for r, d in zip(rows, dims)]
    states = [torch.zeros(r, device=device) for r in rows]
    plan = ops.GroupPlan()
    plan.add_feature(tabs[0], pooling="mean", null_policy="exclude", state=states[0])
    plan.add_feature(tabs[1], pooling="none", state=states[1])
    ln = rng.integers(0, 20, size=B)
    bag = rng.zipf(1.2, size=int(ln.sum())) % rows[0]
    single = rng.zipf(1.2, size=B) % rows[1]
    packed = torch.from_numpy(np.concatenate([bag, single]).astype(np.int64)).to(device)
    lens = torch.from_numpy(np.concatenate([ln, [B]]).astype(np.int64)).to(device)
    out = torch.empty((B, sum(dims)), device=device)
    grad = torch.from_numpy(rng.standard_normal((B, sum(dims))).astype(np.float32)).to(device)
    views = [slice(0, dims[0]), slice(dims[0], sum(dims))]
    st = SparseStep(plan, packed, lens, [bag.size, B], [B, 0], [out[:, v] for v in views],
                    [grad[:, v] for v in views])
    return st, tabs, states, out


def test_sequence_step_rebound_to_longer_rows_matches_oracle(device):
    """A SequenceStep built on short rows, then bound to rows up to the
    window: every position of the longer rows gets its gradient (the packed
    keys are placed each step from the bound lengths)."""
    from mdl_amd.sparse_step import SequenceStep

    rng = np.random.default_rng(85)
    B, L, rows = 48, 160, 6000
    tab = _table(rng, rows, 32, torch.float32, device)
    acc = torch.zeros(rows, device=device)
    plan = ops.GroupPlan()
    plan.add_feature(tab, pooling="none", state=acc)
    out = torch.empty((B, L, 32), device=device)
    mask = torch.empty((B, L), dtype=torch.bool, device=device)
    grad = torch.empty((B, L, 32), device=device)

    def seq(max_len):
        ln = rng.integers(0, max_len + 1, size=B)
        m = np.zeros((B, L), dtype=np.int64)
        for b in range(B):
            k = min(int(ln[b]), L)  # lengths past the input are clamped to it
            m[b, :k] = rng.zipf(1.1, size=k) % rows
        return m, ln

    first = seq(10)
    st = SequenceStep(plan, [torch.from_numpy(first[0]).to(device)], [torch.from_numpy(first[1]).to(device)], [out],
                      [mask], [grad])
    W = to_np(tab).copy()
    A = np.zeros(rows, np.float32)
    for k, (m, ln) in enumerate([first, seq(L), seq(L + 40), seq(60)]):
        announce("sequence_rebind", k, int(np.minimum(ln, L).sum()))
        g = rng.standard_normal((B, L, 32)).astype(np.float32)
        grad.copy_(torch.from_numpy(g))
        st.bind([torch.from_numpy(m).to(device)], [torch.from_numpy(ln).to(device)])
        st.step(0.03, 1e-8)
        assert int(st.count.item()) == int(np.minimum(ln, L).sum())
        ref, rmask = O.sequence_window(W, m, ln, L)
        assert np.array_equal(mask.cpu().numpy(), rmask)
        assert np.array_equal(out.cpu().numpy(), ref)
        r, v = O.sequence_grads(m, ln, g, L)
        rr, vv = O.coalesce(r, v)
        wexp, aexp = O.rowwise_adagrad(W, A, rr, vv, 0.03, 1e-8)
        assert_close(acc.cpu().numpy(), aexp, 1e-5, 1e-7)
        assert_close(to_np(tab), wexp, 1e-5, 1e-6)
        W = to_np(tab).copy()
        A = acc.cpu().numpy().copy()


def test_sequence_step_accumulates_micro_batches(device):
    """SequenceStep(micro_batches=2) over two sequence features sharing no
    table: each micro-batch's windows match the oracle, and one sort + reduce
    applies one row-wise Adagrad step on the coalesced sum of both
    micro-batches' window gradients."""
    from mdl_amd.sparse_step import SequenceStep

    rng = np.random.default_rng(86)
    B, L, k, lr, eps = 40, 96, 2, 0.03, 1e-8
    rows = [5000, 800]
    dims = [32, 16]
    tabs = [_table(rng, r, d, torch.float32, device) for r, d in zip(rows, dims)]
    accs = [torch.from_numpy(rng.random(r).astype(np.float32)).to(device) for r in rows]
    W = [to_np(t).copy() for t in tabs]
    A = [a.cpu().numpy().copy() for a in accs]
    plan = ops.GroupPlan()
    for t, a in zip(tabs, accs):
        plan.add_feature(t, pooling="none", state=a)
    outs = [[torch.empty((B, L, d), device=device) for d in dims] for _ in range(k)]
    masks = [[torch.empty((B, L), dtype=torch.bool, device=device) for _ in dims] for _ in range(k)]
    grads = [[torch.empty((B, L, d), device=device) for d in dims] for _ in range(k)]

    def seq(r, max_len):
        ln = rng.integers(0, max_len + 1, size=B)
        m = np.zeros((B, L), dtype=np.int64)
        for b in range(B):
            n = min(int(ln[b]), L)
            m[b, :n] = rng.zipf(1.1, size=n) % r
        return m, ln

    batches = [[seq(r, mx) for r in rows] for mx in (30, L + 20)]
    st = SequenceStep(plan, [torch.from_numpy(b[0]).to(device) for b in batches[0]],
                      [torch.from_numpy(b[1]).to(device) for b in batches[0]], outs, masks, grads, micro_batches=k)
    g_host = []
    for m, batch in enumerate(batches):
        announce("sequence_micro_batch", m)
        gm = []
        for f, d in enumerate(dims):
            g = rng.standard_normal((B, L, d)).astype(np.float32)
            grads[m][f].copy_(torch.from_numpy(g))
            gm.append(g)
        g_host.append(gm)
        st.bind([torch.from_numpy(b[0]).to(device) for b in batch], [torch.from_numpy(b[1]).to(device) for b in batch])
        st.forward(micro_batch=m)
    st.sort()
    st.apply(lr, eps)
    torch.cuda.synchronize()
    assert int(st.error_count.item()) == 0
    for f in range(len(rows)):
        parts = []
        for m, batch in enumerate(batches):
            ids, ln = batch[f]
            ref, rmask = O.sequence_window(W[f], ids, ln, L)
            assert np.array_equal(masks[m][f].cpu().numpy(), rmask), (m, f)
            assert np.array_equal(outs[m][f].cpu().numpy(), ref), (m, f)
            parts.append(O.sequence_grads(ids, ln, g_host[m][f], L))
        rr, vv = O.coalesce(np.concatenate([p[0] for p in parts]), np.concatenate([p[1] for p in parts]))
        wexp, aexp = O.rowwise_adagrad(W[f], A[f], rr, vv, lr, eps)
        assert_close(accs[f].cpu().numpy(), aexp, 1e-5, 1e-7)
        assert_close(to_np(tabs[f]), wexp, 1e-5, 1e-6)
    with pytest.raises(ValueError):
        st.step(lr, eps)


@pytest.mark.parametrize("clip", [None, 0.5])
def test_sparse_step_graph_replays_match_eager(device, clip):
    """Every replay of a captured step equals an eager step bit for bit, with
    eager work and synchronisations between the replays (the step records no
    memset: its counters and flags are written by kernels)."""
    announce("graph_replay", clip)
    eager, tabs_e, states_e, out_e = _slot_step(device, 92)
    graph, tabs_g, states_g, out_g = _slot_step(device, 92)
    lr, eps = 0.05, 1e-8
    eager.step(lr, eps, clip)
    graph.step(lr, eps, clip)  # loads the kernels before the recording
    graph.capture(lr, eps, clip)
    for r in range(4):
        eager.step(lr, eps, clip)
        graph.replay()
        torch.cuda.synchronize()
        _ = float((tabs_g[0].double() * 2).sum())  # eager work between replays
        assert torch.equal(out_g, out_e), f"replay {r}: outputs"
        for t in range(2):
            assert torch.equal(tabs_g[t], tabs_e[t]), f"replay {r}: table {t}"
            assert torch.equal(states_g[t], states_e[t]), f"replay {r}: state {t}"


def test_sequence_step_graph_replays_match_eager(device):
    """A captured SequenceStep replays bit-identically to eager steps."""
    from mdl_amd.sparse_step import SequenceStep

    announce("sequence_graph_replay")

    def build():
        rng = np.random.default_rng(93)
        B, L, rows = 32, 128, 5000
        tab = _table(rng, rows, 64, torch.float32, device)
        acc = torch.zeros(rows, device=device)
        plan = ops.GroupPlan()
        plan.add_feature(tab, pooling="none", state=acc)
        ln = rng.integers(0, L + 1, size=B)
        m = np.zeros((B, L), dtype=np.int64)
        for b in range(B):
            m[b, : ln[b]] = rng.zipf(1.05, size=ln[b]) % rows
        out = torch.empty((B, L, 64), device=device)
        mask = torch.empty((B, L), dtype=torch.bool, device=device)
        grad = torch.from_numpy(rng.standard_normal((B, L, 64)).astype(np.float32)).to(device)
        st = SequenceStep(plan, [torch.from_numpy(m).to(device)], [torch.from_numpy(ln).to(device)], [out], [mask],
                          [grad])
        return st, tab, acc, out

    eager, tab_e, acc_e, out_e = build()
    graph, tab_g, acc_g, out_g = build()
    eager.step(0.02, 1e-8)
    graph.step(0.02, 1e-8)
    graph.capture(0.02, 1e-8)
    for r in range(3):
        eager.step(0.02, 1e-8)
        graph.replay()
        torch.cuda.synchronize()
        _ = float(acc_g.double().sum())  # eager work between replays
        assert torch.equal(out_g, out_e), f"replay {r}: window"
        assert torch.equal(tab_g, tab_e), f"replay {r}: table"
        assert torch.equal(acc_g, acc_e), f"replay {r}: state"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("dim", [3, 16, 64, 130, 300])
def test_single_id_bags_match_oracle(device, dtype, dim):
    """Pooled features whose bags hold one id each (c4's) take a gather
    instead of the pooled walk: each output row is its id's row bit for bit
    (zeros for a null under "exclude" and for ids outside the table), the bag
    weights feed the mean's backward, and a feature with one two-id bag per
    chunk takes the walk on the same ids.  Sum and mean, both null policies,
    through the fused step against the oracle."""

    from mdl_amd.sparse_step import SparseStep

    announce("single_id_bags", dtype, dim)
    rng = np.random.default_rng(95 + dim)
    B, rows = 2000, 5000
    bf16 = dtype == torch.bfloat16
    cases = [("sum", "exclude", False), ("mean", "exclude", False), ("mean", "include_as_padding", False),
             ("sum", "include_as_padding", False), ("mean", "exclude", True)]
    W0 = [rng.standard_normal((rows, dim)).astype(np.float32) for _ in cases]
    if bf16:
        W0 = [torch.from_numpy(w).to(torch.bfloat16).float().numpy() for w in W0]
    tabs = [torch.from_numpy(w).to(dtype).to(device) for w in W0]
    A0 = [rng.random(rows).astype(np.float32) for _ in cases]
    accs = [torch.from_numpy(a.copy()).to(device) for a in A0]
    plan = ops.GroupPlan()
    ids, lens = [], []
    for t, (mode, pol, two) in enumerate(cases):
        plan.add_feature(tabs[t], pooling=mode, null_policy=pol, state=accs[t])
        ln = np.ones(B, dtype=np.int64)
        if two:
            ln[::97] = 2  # one two-id bag in most chunks: the walk
        x = (rng.zipf(1.2, size=int(ln.sum())) - 1) % rows
        x[rng.random(x.size) < 0.05] = 0
        x[rng.random(x.size) < 0.01] = rows + 3
        ids.append(x.astype(np.int64))
        lens.append(ln)
    S = dim * len(cases)
    outs = [torch.empty((B, dim), dtype=dtype, device=device) for _ in cases]
    g_slot = rng.standard_normal((B, S))
    grads = []
    for t in range(len(cases)):
        g = torch.from_numpy(g_slot[:, t * dim: (t + 1) * dim].astype(np.float32)).to(dtype)
        g_slot[:, t * dim: (t + 1) * dim] = g.double().numpy()
        grads.append(g.to(device))
    err = torch.zeros(1, dtype=torch.int32, device=device)
    st = SparseStep(plan, torch.from_numpy(np.concatenate(ids)).to(device),
                    torch.from_numpy(np.concatenate(lens)).to(device), [x.size for x in ids], [B] * len(cases),
                    outs, grads, error_count=err)
    st.step(0.03, 1e-8)
    torch.cuda.synchronize()
    feats, offs, bag_off, ids_off = [], [], 0, 0
    for t, ((mode, pol, _), x, ln) in enumerate(zip(cases, ids, lens)):
        feats.append({"table": t, "pooling": 1 if mode == "sum" else 2, "exclude": int(pol == "exclude"),
                      "ids_off": ids_off, "bag_off": bag_off, "num_bags": B, "out_col": t * dim})
        o = O.offsets_of(ln)
        offs.append(o)
        bag_off += len(o)
        ids_off += x.size
    tables = [{"W": w.copy(), "acc": a.copy(), "is_bf16": bf16} for w, a in zip(W0, A0)]
    ref = O.sparse_step(feats, tables, np.concatenate(ids), np.concatenate(offs), S, g_slot, 0.03, 1e-8)
    assert int(err.item()) == sum(int((x >= rows).sum()) for x in ids)
    for t, (mode, pol, two) in enumerate(cases):
        got = outs[t].float().cpu().numpy()
        want = ref[:, t * dim: (t + 1) * dim]
        if two:
            assert_close(got, want, RTOL[dtype], 1e-6 if not bf16 else 1e-2)
        else:
            assert np.array_equal(got, want.astype(np.float32)), f"{mode}/{pol} output"
        assert_close(tabs[t].float().cpu().numpy(), tables[t]["W"], RTOL[dtype], 1e-6 if not bf16 else 1e-2)
        assert_close(accs[t].cpu().numpy(), tables[t]["acc"], 1e-5, 1e-7)
