"""Plans of more than 2^32 - 1 rows on one GPU: key groups.

Two dim-8 bf16 tables of 2.2e9 and 2.3e9 rows and a small fp32 table (about
4.5e9 rows, 72 GB of weights and 18 GB of accumulators) are more rows than one
32-bit key space holds, so the plan is cut into two key groups: the first
table's features, then the second's and the third's.  These paths run over
them and are checked against the CPU oracle on compact copies of the touched
rows (rows above 2^31 of a table and keys above 2^31 of a group included):

* ``SparseStep`` (bag lengths placed on the device, each group's keys placed
  by its key origin), with the clip norm summed over both groups; its form
  without pooled features (host-known origins); two accumulated
  micro-batches;
* the ``mdl_hip::grouped_lookup`` custom op and its backward (the drop-in's
  path), with a feature order that reads the first table again after the
  second, so the op must reorder its features by table;
* ``ops.grouped_forward`` + ``ops.backward_adagrad`` with a clip that scales
  the gradient of both groups by one coefficient;
* the drop-in modules (``ShardedEmbedding`` lookups, ``loss.backward()``,
  ``ShardedRowWiseAdagrad.step()``).

Untouched rows and accumulators of every table are checked bit for bit
(checksums) after every SparseStep.
"""

import time

import numpy as np
import pytest
import torch

from mdl_amd import ops
from mdl_amd.sparse_step import SparseStep
from oracle import oracle as O
from parity_helpers import RTOL, _check_update, _free, _random_state, _Snapshot, _touched, assert_close, say

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(900)]

ROWS = [2_200_000_000, 2_300_000_000, 10_000]
DIMS = [8, 8, 16]
DTYPES = [torch.bfloat16, torch.bfloat16, torch.float32]
LR, EPS = 0.05, 1e-8
B = 2048


@pytest.fixture(scope="module")
def big(device):
    t0 = time.time()
    say("key_groups", "allocating", f"{sum(ROWS):.3e} rows")
    tables = [torch.empty((r, d), dtype=dt, device=device) for r, d, dt in zip(ROWS, DIMS, DTYPES)]
    states = [torch.empty(r, dtype=torch.float32, device=device) for r in ROWS]
    _random_state(states, 11)
    torch.cuda.synchronize()
    say("key_groups", "tables ready", f"{time.time() - t0:.1f}s")
    yield tables, states
    del tables, states
    _free()


def _draw(rng, feats):
    """Ids (uniform over the table, a hot set with the edge rows, and nulls)
    and bag lengths of each (table, pooling) feature."""

    ids, lens = [], []
    for t, pool in feats:
        R = ROWS[t]
        if pool == "none":
            ln, n = None, B
        else:
            ln = rng.integers(0, 16, size=B)
            n = int(ln.sum())
        x = rng.integers(0, R, size=n)
        edge = np.array([R - 1, R - 2, min(1 << 31, R - 1), min((1 << 31) - 1, R - 1), 1, 2], dtype=np.int64)
        hot = np.concatenate([edge, rng.integers(0, R, size=300)])
        pick = rng.random(n)
        x[pick < 0.3] = rng.choice(hot, size=int((pick < 0.3).sum()))
        x[pick > 0.93] = 0
        ids.append(x.astype(np.int64))
        lens.append(ln)
    return ids, lens


def _set_touched(tables, touched, rng):
    """Random values in the touched rows (the rest of a table is whatever
    the allocation held: the checks read it only through checksums)."""

    for w, u in zip(tables, touched):
        vals = torch.from_numpy(rng.standard_normal((u.size, w.size(1))).astype(np.float32)).to(w.device)
        w.index_copy_(0, torch.from_numpy(u).to(w.device), vals.to(w.dtype))


def _oracle_grads(feats, ids, lens, grads, touched, snap, outs, what):
    """Check every output; per table the coalesced gradient (rows in the
    compact numbering, fp64 sums) and the same sums over |terms|."""

    return _coalesced(_oracle_parts(feats, ids, lens, grads, touched, snap, outs, what))


def _coalesced(parts):
    rows_t, vals_t, absv_t = parts
    out = []
    for t in range(len(ROWS)):
        if not rows_t[t]:
            out.append(None)
            continue
        rr, g = O.coalesce(np.concatenate(rows_t[t]), np.concatenate(vals_t[t]))
        _, s = O.coalesce(np.concatenate(rows_t[t]), np.concatenate(absv_t[t]))
        out.append((rr, g, s))
    return out


def _oracle_parts(feats, ids, lens, grads, touched, snap, outs, what):
    """Check every output; per table the per-id gradients (compact rows,
    fp64 values, |values|) of one batch."""

    T = len(ROWS)
    rows_t = [[] for _ in range(T)]
    vals_t = [[] for _ in range(T)]
    absv_t = [[] for _ in range(T)]
    for f, ((t, pool), x, ln) in enumerate(zip(feats, ids, lens)):
        lid = np.searchsorted(touched[t], x)
        got = outs[f].float().cpu().numpy()
        gf = grads[f].float().cpu().numpy().astype(np.float64)
        rtol = RTOL["fp32" if DTYPES[t] == torch.float32 else "bf16"]
        if pool == "none":
            assert np.array_equal(got, snap.w[t][lid]), f"{what} feature {f}: gathered rows"
            r, v = O.per_id_grads(lid, None, gf, "none", "exclude")
            _, va = O.per_id_grads(lid, None, np.abs(gf), "none", "exclude")
        else:
            ref, _ = O.pool(snap.w[t], lid, ln, pool, "exclude")
            mag, _ = O.pool(np.abs(snap.w[t]), lid, ln, pool, "exclude")
            assert_close(got, ref, rtol, 1e-7, mag, f"{what} feature {f} pooled")
            r, v = O.per_id_grads(lid, ln, gf, pool, "exclude")
            _, va = O.per_id_grads(lid, ln, np.abs(gf), pool, "exclude")
        rows_t[t].append(r)
        vals_t[t].append(v)
        absv_t[t].append(va)
    return rows_t, vals_t, absv_t


def _touched_of(feats, ids):
    per = [[] for _ in ROWS]
    for (t, _), x in zip(feats, ids):
        per[t].append(x)
    return [_touched(xs) if xs else np.zeros(1, np.int64) for xs in per]


def _plan(tables, states, feats):
    plan = ops.GroupPlan()
    for t, pool in feats:
        plan.add_feature(tables[t], pooling=pool, null_policy="exclude", state=states[t])
    return plan


def _grads(rng, outs):
    return [torch.from_numpy(rng.standard_normal(tuple(o.shape)).astype(np.float32)).to(o.device).to(o.dtype)
            for o in outs]


def test_sparse_step_over_two_key_groups_matches_oracle(device, big):
    t0 = time.time()
    tables, states = big
    rng = np.random.default_rng(4500)
    feats = [(0, "mean"), (0, "none"), (1, "sum"), (2, "none")]
    plan = _plan(tables, states, feats)
    assert plan.split and [(g.lo, g.hi, g.tables) for g in plan.groups] == [(0, 2, [0]), (2, 4, [1, 2])]
    assert plan.key_bits == 32
    ids, lens = _draw(rng, feats)
    touched = _touched_of(feats, ids)
    _set_touched(tables, touched, rng)
    snap = _Snapshot(tables, states, touched, device)
    say("key_groups", "sparse step snapshot", f"{time.time() - t0:.1f}s")
    outs = [torch.empty((B if ln is not None else x.size, DIMS[t]), dtype=DTYPES[t], device=device)
            for (t, _), x, ln in zip(feats, ids, lens)]
    grads = _grads(rng, outs)
    packed = torch.from_numpy(np.concatenate(ids)).to(device)
    lengths = torch.from_numpy(np.concatenate(
        [ln if ln is not None else np.array([x.size]) for x, ln in zip(ids, lens)]).astype(np.int64)).to(device)
    st = SparseStep(plan, packed, lengths, [x.size for x in ids], [0 if ln is None else B for ln in lens],
                    outs, grads)
    assert len(st.groups) == 2
    st.forward()
    st.sort()
    norm, coef = st.clip(1e9)
    st.apply(LR, EPS, coef)
    torch.cuda.synchronize()
    assert int(st.error_count.item()) == 0
    say("key_groups", "sparse step done", f"{time.time() - t0:.1f}s")
    w_post, a_post = snap.after(tables, states)
    ref = _oracle_grads(feats, ids, lens, grads, touched, snap, outs, "sparse step")
    sumsq = 0.0
    for t, r in enumerate(ref):
        rr, g, s = r
        sumsq += float((g * g).sum())
        bf = DTYPES[t] == torch.bfloat16
        _check_update(f"sparse step table {t}", w_post[t], a_post[t], snap.w[t], snap.a[t], rr, g, s, LR, EPS,
                      RTOL["bf16" if bf else "fp32"], 1e-6 if bf else 1e-7, bf)
    assert_close(norm.cpu().numpy(), np.array([np.sqrt(sumsq)]), 1e-4, 0, what="clip norm")
    say("key_groups", "sparse step checked", f"{time.time() - t0:.1f}s")
    snap.restore_and_check(tables, states)
    say("key_groups", "untouched rows checked", f"{time.time() - t0:.1f}s")


@pytest.mark.parametrize("case", ["unpooled", "micro_batches"])
def test_sparse_step_forms_over_two_key_groups(device, big, case):
    """SparseStep over the two key groups in its other forms: a layout
    without pooled features (ids placed by host-known counts, each group's
    origin and count uploaded once), and two micro-batches of a pooled layout
    accumulated into one update."""

    t0 = time.time()
    tables, states = big
    rng = np.random.default_rng(4510 if case == "unpooled" else 4511)
    if case == "unpooled":
        feats = [(0, "none"), (1, "none"), (2, "none")]
        k = 1
    else:
        feats = [(0, "mean"), (1, "sum"), (2, "none")]
        k = 2
    plan = _plan(tables, states, feats)
    assert [(g.lo, g.hi) for g in plan.groups] == [(0, 1), (1, 3)]
    draws = [_draw(rng, feats) for _ in range(k)]
    per = [[] for _ in ROWS]
    for ids, _ in draws:
        for (t, _), x in zip(feats, ids):
            per[t].append(x)
    touched = [_touched(xs) for xs in per]
    _set_touched(tables, touched, rng)
    snap = _Snapshot(tables, states, touched, device)
    outs = [[torch.empty((B if ln is not None else x.size, DIMS[t]), dtype=DTYPES[t], device=device)
             for (t, _), x, ln in zip(feats, ids, lens)] for ids, lens in draws]
    grads = [_grads(rng, o) for o in outs]
    packed = [torch.from_numpy(np.concatenate(ids)).to(device) for ids, _ in draws]
    lengths = [None if case == "unpooled" else torch.from_numpy(np.concatenate(
        [ln if ln is not None else np.array([x.size]) for x, ln in zip(ids, lens)]).astype(np.int64)).to(device)
        for ids, lens in draws]
    ids0, lens0 = draws[0]
    st = SparseStep(plan, packed[0], lengths[0], [x.size for x in ids0], [0 if ln is None else B for ln in lens0],
                    outs[0] if k == 1 else outs, grads[0] if k == 1 else grads,
                    capacity=max(int(p.numel()) for p in packed), micro_batches=k)
    assert len(st.groups) == 2
    for m in range(k):
        st.bind(packed[m], lengths[m])
        st.forward(micro_batch=m)
    st.sort()
    st.apply(LR, EPS)
    torch.cuda.synchronize()
    assert int(st.error_count.item()) == 0
    say("key_groups", case, "step done", f"{time.time() - t0:.1f}s")
    w_post, a_post = snap.after(tables, states)
    parts = [[] for _ in range(3)]
    for m, (ids, lens) in enumerate(draws):
        got = _oracle_parts(feats, ids, lens, grads[m], touched, snap, outs[m], f"{case} micro-batch {m}")
        for j in range(3):
            parts[j].append(got[j])
    merged = tuple([sum((p[t] for p in parts[j]), []) for t in range(len(ROWS))] for j in range(3))
    for t, (rr, g, s) in enumerate(_coalesced(merged)):
        bf = DTYPES[t] == torch.bfloat16
        _check_update(f"{case} table {t}", w_post[t], a_post[t], snap.w[t], snap.a[t], rr, g, s, LR, EPS,
                      RTOL["bf16" if bf else "fp32"], 1e-6 if bf else 1e-7, bf)
    snap.restore_and_check(tables, states)
    say("key_groups", case, "checked", f"{time.time() - t0:.1f}s")


def test_grouped_lookup_op_reorders_features_across_key_groups(device, big):
    """The drop-in's op: features [t0 mean, t1 sum, t0 none, t2 none] read
    table 0 again after table 1; outputs come back in the caller's order and
    the coalesced gradients of every table match the oracle."""

    t0 = time.time()
    tables, states = big
    rng = np.random.default_rng(4501)
    feats = [(0, "mean"), (1, "sum"), (0, "none"), (2, "none")]
    ids, lens = _draw(rng, feats)
    touched = _touched_of(feats, ids)
    _set_touched(tables, touched, rng)
    snap = _Snapshot.__new__(_Snapshot)
    snap.idx = [torch.from_numpy(u).to(device) for u in touched]
    snap.w = [w.index_select(0, i).float().cpu().numpy() for w, i in zip(tables, snap.idx)]
    code = {"none": 0, "sum": 1, "mean": 2}
    ids_dev = [torch.from_numpy(x).to(device) for x in ids]
    lens_dev = [None if ln is None else torch.from_numpy(ln).to(device) for ln in lens]
    outs, keys, payload, bag_count, offsets, err = torch.ops.mdl_hip.grouped_lookup(
        tables, ids_dev, lens_dev, [t for t, _ in feats], [code[p] for _, p in feats], [1] * 4, [0] * 4, True)
    grads = _grads(rng, outs)
    rows_all, vbuf, counts = torch.ops.mdl_hip.grouped_lookup_backward(
        tables, ids_dev, lens_dev, [t for t, _ in feats], [code[p] for _, p in feats], [1] * 4, [0] * 4, grads,
        keys, payload, bag_count, offsets)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    say("key_groups", "op done", f"{time.time() - t0:.1f}s")
    cap = [0, 0, 0]
    for (t, _), x in zip(feats, ids):
        cap[t] += x.size
    rows, values = ops.split_coalesced(tables, rows_all, vbuf, ops.coalesced_layout(tables, cap))
    ref = _oracle_grads(feats, ids, lens, grads, touched, snap, outs, "op")
    counts = counts.cpu().numpy()
    for t, (rr, g, s) in enumerate(ref):
        u = int(counts[t])
        assert u == rr.size, f"op table {t}: {u} rows, oracle {rr.size}"
        got_rows = rows[t].cpu().numpy()
        assert np.array_equal(got_rows[:u], touched[t][rr]), f"op table {t}: rows"
        got = values[t].float().cpu().numpy()
        rtol = RTOL["fp32" if DTYPES[t] == torch.float32 else "bf16"]
        assert_close(got[:u], g, rtol, 1e-6, s, f"op table {t} values")
        # capacity padding: the last row again, zero values
        assert (got_rows[u:] == got_rows[u - 1]).all() and not got[u:].any()
    say("key_groups", "op checked", f"{time.time() - t0:.1f}s")


def test_functional_backward_adagrad_clips_across_key_groups(device, big):
    t0 = time.time()
    tables, states = big
    rng = np.random.default_rng(4502)
    feats = [(0, "sum"), (1, "mean"), (1, "none"), (2, "mean")]
    plan = _plan(tables, states, feats)
    assert [(g.lo, g.hi) for g in plan.groups] == [(0, 1), (1, 4)]
    ids, lens = _draw(rng, feats)
    touched = _touched_of(feats, ids)
    _set_touched(tables, touched, rng)
    snap = _Snapshot.__new__(_Snapshot)
    snap.idx = [torch.from_numpy(u).to(device) for u in touched]
    snap.w = [w.index_select(0, i).float().cpu().numpy() for w, i in zip(tables, snap.idx)]
    snap.a = [a.index_select(0, i).cpu().numpy() for a, i in zip(states, snap.idx)]
    ids_dev = [torch.from_numpy(x).to(device) for x in ids]
    lens_dev = [None if ln is None else torch.from_numpy(ln).to(device) for ln in lens]
    res = ops.grouped_forward(plan, ids_dev, lens_dev, with_backward=True)
    outs = res.outputs
    grads = _grads(rng, outs)
    ref = _oracle_grads(feats, ids, lens, grads, touched, snap, outs, "functional")
    norm_ref = float(np.sqrt(sum(float((g * g).sum()) for _, g, _ in ref)))
    clip = 0.3 * norm_ref
    norm = ops.backward_adagrad(res, grads, lr=LR, eps=EPS, clip_norm=clip)
    torch.cuda.synchronize()
    say("key_groups", "functional step done", f"{time.time() - t0:.1f}s")
    assert_close(norm.cpu().numpy(), np.array([norm_ref]), 1e-4, 0, what="clip norm")
    coef = min(clip / (norm_ref + 1e-6), 1.0)
    w_post, a_post = snap.after(tables, states)
    for t, (rr, g, s) in enumerate(ref):
        bf = DTYPES[t] == torch.bfloat16
        _check_update(f"functional table {t}", w_post[t], a_post[t], snap.w[t], snap.a[t], rr, g * coef,
                      s * coef + np.abs(g) * 1e-4, LR, EPS, RTOL["bf16" if bf else "fp32"], 1e-6 if bf else 1e-7, bf)
    say("key_groups", "functional step checked", f"{time.time() - t0:.1f}s")


def test_dropin_modules_train_across_key_groups(device, big):
    """ShardedEmbedding modules over the three tables and ShardedRowWiseAdagrad:
    a pooled call over tables 0 and 1 (4.5e9 rows: two key groups) and an
    unpooled call over tables 0 and 2, loss.backward() (table 0's two sparse
    gradients accumulate), opt.step() -- every touched row and accumulator
    against one oracle update of each table's coalesced gradient."""

    from torch import nn

    from mdl_amd.embeddings import (EmbeddingShardSpec, ShardedEmbedding, grouped_sharded_embedding_lookup,
                                    pooled_embedding_lookup)
    from mdl_amd.optim import ShardedRowWiseAdagrad

    t0 = time.time()
    tables, states = big
    rng = np.random.default_rng(4503)
    mods = []
    for t, w in enumerate(tables):
        spec = EmbeddingShardSpec(table_name=f"kg_{t}", strategy="row_wise", world_size=1)
        m = ShardedEmbedding(2, int(w.size(1)), table_name=f"kg_{t}", shard_spec=spec, collect_stats=False,
                             dtype=w.dtype).to(device)
        m.weight = nn.Parameter(w)
        m.num_embeddings = int(w.size(0))
        mods.append(m)
    opt = ShardedRowWiseAdagrad([m.weight for m in mods], lr=LR, eps=EPS)
    for m, a in zip(mods, states):
        opt.state[m.weight]["sum"] = a
    feats = [(0, "mean"), (1, "sum"), (0, "none"), (2, "none")]
    ids, lens = _draw(rng, feats)
    touched = _touched_of(feats, ids)
    _set_touched(tables, touched, rng)
    snap = _Snapshot.__new__(_Snapshot)
    snap.idx = [torch.from_numpy(u).to(device) for u in touched]
    snap.w = [w.index_select(0, i).float().cpu().numpy() for w, i in zip(tables, snap.idx)]
    snap.a = [a.index_select(0, i).cpu().numpy() for a, i in zip(states, snap.idx)]
    x = [torch.from_numpy(v).to(device) for v in ids]
    pooled = pooled_embedding_lookup([(mods[0], x[0], torch.from_numpy(lens[0]).to(device), "mean", "exclude"),
                                      (mods[1], x[1], torch.from_numpy(lens[1]).to(device), "sum", "exclude")])
    single = grouped_sharded_embedding_lookup([(mods[0], x[2]), (mods[2], x[3])])
    outs = pooled + single
    grads = _grads(rng, outs)
    torch.autograd.backward(outs, grads)
    opt.step()
    torch.cuda.synchronize()
    say("key_groups", "drop-in step done", f"{time.time() - t0:.1f}s")
    w_post, a_post = snap.after(tables, states)
    ref = _oracle_grads(feats, ids, lens, grads, touched, snap, [o.detach() for o in outs], "drop-in")
    for t, (rr, g, s) in enumerate(ref):
        # the drop-in's sparse gradients are stored in the table's dtype, as
        # the reference's are: bf16 tables take the bf16 tolerance for state
        bf = DTYPES[t] == torch.bfloat16
        _check_update(f"drop-in table {t}", w_post[t], a_post[t], snap.w[t], snap.a[t], rr, g, s, LR, EPS,
                      RTOL["bf16" if bf else "fp32"], 1e-6 if bf else 1e-7, bf,
                      acc_rtol=RTOL["bf16" if bf else "fp32"])
    say("key_groups", "drop-in step checked", f"{time.time() - t0:.1f}s")
    for m in mods:
        m.weight = None
    del opt, mods


@pytest.mark.parametrize("order", ["oldest_to_newest", "newest_to_oldest"])
def test_sequence_step_over_two_key_groups_matches_oracle(device, big, order):
    """SequenceStep over the 4.5e9-row plan: one sequence feature per table,
    so the first table's feature is one key group and the other two features
    the second.  Each group packs its entries into its own key buffer, placed
    by a scan over its own rows, and is sorted and reduced apart.  Windows,
    masks and the touched rows' update against the oracle."""

    from mdl_amd.sparse_step import SequenceStep

    t0 = time.time()
    tables, states = big
    rng = np.random.default_rng(4600 + (order == "newest_to_oldest"))
    Bs, L_in, L_out = 96, 120, 100
    plan = ops.GroupPlan()
    for t in range(3):
        plan.add_feature(tables[t], pooling="none", state=states[t])
    assert plan.split and [(g.lo, g.hi) for g in plan.groups] == [(0, 1), (1, 3)]
    ids, lens = [], []
    for t in range(3):
        R = ROWS[t]
        ln = rng.integers(0, L_in + 1, size=Bs)
        hot = np.concatenate([[R - 1, R - 2, min(1 << 31, R - 1), 1], rng.integers(0, R, size=200)])
        m = np.where(rng.random((Bs, L_in)) < 0.4, rng.choice(hot, size=(Bs, L_in)),
                     rng.integers(0, R, size=(Bs, L_in)))
        m[rng.random((Bs, L_in)) > 0.95] = 0
        m[np.arange(L_in)[None, :] >= ln[:, None]] = 0
        ids.append(m.astype(np.int64))
        lens.append(ln)
    touched = [_touched(m) for m in ids]
    _set_touched(tables, touched, rng)
    snap = _Snapshot(tables, states, touched, device)
    outs = [torch.empty((Bs, L_out, DIMS[t]), dtype=DTYPES[t], device=device) for t in range(3)]
    masks = [torch.empty((Bs, L_out), dtype=torch.bool, device=device) for _ in range(3)]
    grads = _grads(rng, outs)
    st = SequenceStep(plan, [torch.from_numpy(m).to(device) for m in ids],
                      [torch.from_numpy(ln).to(device) for ln in lens], outs, masks, grads, order=order)
    assert len(st.groups) == 2
    st.step(LR, EPS)
    torch.cuda.synchronize()
    assert int(st.error_count.item()) == 0
    assert int(st.count.item()) == sum(int(np.minimum(ln, L_out).sum()) for ln in lens)
    say("key_groups", "sequence step done", order, f"{time.time() - t0:.1f}s")
    w_post, a_post = snap.after(tables, states)
    for t in range(3):
        mask, src = O.sequence_positions(ids[t], lens[t], L_out, order)
        assert np.array_equal(masks[t].cpu().numpy(), mask), f"table {t} mask"
        lid = np.searchsorted(touched[t], ids[t])
        rows_at = np.take_along_axis(lid, src, axis=1)
        got = outs[t].float().cpu().numpy()
        assert np.array_equal(got[mask], snap.w[t][rows_at[mask]]), f"table {t} window rows"
        assert not got[~mask].any(), f"table {t} window padding"
        g = grads[t].float().cpu().numpy().astype(np.float64)
        live = mask & (np.take_along_axis(ids[t], src, axis=1) != 0)
        rr, gg = O.coalesce(rows_at[live], g[live])
        _, ss = O.coalesce(rows_at[live], np.abs(g[live]))
        bf = DTYPES[t] == torch.bfloat16
        _check_update(f"sequence step table {t}", w_post[t], a_post[t], snap.w[t], snap.a[t], rr, gg, ss, LR, EPS,
                      RTOL["bf16" if bf else "fp32"], 1e-6 if bf else 1e-7, bf)
    snap.restore_and_check(tables, states)
    say("key_groups", "sequence step checked", order, f"{time.time() - t0:.1f}s")


def test_sequence_step_micro_batches_over_two_key_groups(device, big):
    """SequenceStep(micro_batches=2) over the 4.5e9-row plan: each key group
    holds both micro-batches' window entries in regions of its key buffer,
    and one sort + reduce per group applies one row-wise Adagrad step on the
    coalesced sum of both micro-batches' window gradients."""

    from mdl_amd.sparse_step import SequenceStep

    t0 = time.time()
    tables, states = big
    rng = np.random.default_rng(4700)
    k, Bs, L_in, L_out = 2, 64, 90, 80
    plan = ops.GroupPlan()
    for t in range(3):
        plan.add_feature(tables[t], pooling="none", state=states[t])

    def batch(max_len):
        ids, lens = [], []
        for t in range(3):
            R = ROWS[t]
            ln = rng.integers(0, max_len + 1, size=Bs)
            hot = np.concatenate([[R - 1, min(1 << 31, R - 1), 2], rng.integers(0, R, size=100)])
            m = np.where(rng.random((Bs, L_in)) < 0.5, rng.choice(hot, size=(Bs, L_in)),
                         rng.integers(0, R, size=(Bs, L_in)))
            m[np.arange(L_in)[None, :] >= ln[:, None]] = 0
            ids.append(m.astype(np.int64))
            lens.append(ln)
        return ids, lens

    batches = [batch(40), batch(L_in)]
    touched = [_touched([b[0][t] for b in batches]) for t in range(3)]
    _set_touched(tables, touched, rng)
    snap = _Snapshot(tables, states, touched, device)
    outs = [[torch.empty((Bs, L_out, DIMS[t]), dtype=DTYPES[t], device=device) for t in range(3)] for _ in range(k)]
    masks = [[torch.empty((Bs, L_out), dtype=torch.bool, device=device) for _ in range(3)] for _ in range(k)]
    grads = [_grads(rng, o) for o in outs]
    dev = [([torch.from_numpy(m).to(device) for m in ids], [torch.from_numpy(ln).to(device) for ln in lens])
           for ids, lens in batches]
    st = SequenceStep(plan, dev[0][0], dev[0][1], outs, masks, grads, micro_batches=k)
    assert len(st.groups) == 2
    for m in range(k):
        st.bind(*dev[m])
        st.forward(micro_batch=m)
    st.sort()
    st.apply(LR, EPS)
    torch.cuda.synchronize()
    assert int(st.error_count.item()) == 0
    say("key_groups", "sequence micro-batches done", f"{time.time() - t0:.1f}s")
    w_post, a_post = snap.after(tables, states)
    for t in range(3):
        rows, vals, absv = [], [], []
        for m, (ids, lens) in enumerate(batches):
            mask, src = O.sequence_positions(ids[t], lens[t], L_out)
            assert np.array_equal(masks[m][t].cpu().numpy(), mask), (m, t)
            r, v = O.sequence_grads(ids[t], lens[t], grads[m][t].float().cpu().numpy(), L_out)
            rows.append(np.searchsorted(touched[t], r))
            vals.append(v)
            absv.append(np.abs(v))
        rr, gg = O.coalesce(np.concatenate(rows), np.concatenate(vals))
        _, ss = O.coalesce(np.concatenate(rows), np.concatenate(absv))
        bf = DTYPES[t] == torch.bfloat16
        _check_update(f"sequence micro-batches table {t}", w_post[t], a_post[t], snap.w[t], snap.a[t], rr, gg, ss,
                      LR, EPS, RTOL["bf16" if bf else "fp32"], 1e-6 if bf else 1e-7, bf)
    snap.restore_and_check(tables, states)
    say("key_groups", "sequence micro-batches checked", f"{time.time() - t0:.1f}s")
