"""Parity of one fused step at every BASELINE configuration's full size.

Each test builds the bench's own workload (the table sizes, id streams and
output layout that ``bench.py`` times), runs one step through the product
(``SparseStep`` / ``SequenceStep`` over the C ABI) and checks it against the
CPU oracle:

* every output row: gathered rows and masks bit for bit, pooled rows within
  the stated tolerance of the same sum over |terms|;
* every touched weight row and accumulator after the update;
* every untouched row of every table (and its accumulator) bit for bit: a
  checksum of each table before the step equals the checksum after the step
  once the touched rows are put back.

The oracle runs on compact copies of the touched rows: a table's ids are
remapped to their rank among its distinct ids, with the padding row 0 first,
which preserves every value the step reads or writes.  Accumulators start
from random non-negative values so the update reads real state.

Tolerances (the path's specification: 1e-5 relative for fp32 storage, 1e-2
for bf16 storage with fp32 accumulation) are applied to first-order error
bounds of fp32 summation: a sum of many terms is compared relative to the
same sum over |terms|, and the accumulator and the updated weight inherit
that bound through the update formula (see ``_check_update``).

The tests free their tables at the end (c1 and c2 do not fit together) and
print their progress, since each takes tens of seconds.
"""

import time

import numpy as np
import pytest
import torch

import bench
from oracle import oracle as O
from parity_helpers import RTOL, STATS, _check_update, _free, _random_state, _Snapshot, _touched, assert_close, say

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(900)]

@pytest.mark.parametrize("name", ["c0", "c4", "c1", "c3"])
def test_pooled_config_full_size_matches_oracle(device, name):
    t0 = time.time()
    wl = bench.WORKLOADS[name]()
    say(name, "drawing batch", f"{len(wl.features)} features, {sum(wl.rows):.3e} rows, batch {wl.batch}")
    rng = np.random.default_rng(1000 + int(name[1]))
    ids, lengths = bench.draw_batch(rng, wl)
    dev = bench.DeviceStep(wl, [(ids, lengths)], device)
    try:
        _random_state(dev.states, 5)
        T = len(wl.rows)
        per_table = [[] for _ in range(T)]
        for f, x in zip(wl.features, ids):
            per_table[f.table].append(x)
        touched = [_touched(xs) for xs in per_table]
        snap = _Snapshot(dev.tables, dev.states, touched, device)
        torch.cuda.synchronize()
        say(name, "tables ready", f"{time.time() - t0:.1f}s", f"{sum(u.size for u in touched)} touched rows")
        dev.step(0)
        torch.cuda.synchronize()
        assert int(dev.err.item()) == 0
        say(name, "step done", f"{time.time() - t0:.1f}s")
        w_post, a_post = snap.after(dev.tables, dev.states)
        out = dev.out.float().cpu().numpy()
        grad = dev.grad.float().cpu().numpy()
        rtol = RTOL[wl.dtype]
        cols = np.concatenate([[0], np.cumsum([wl.dims[f.table] for f in wl.features])[:-1]])
        rows_t = [[] for _ in range(T)]
        vals_t = [[] for _ in range(T)]
        absv_t = [[] for _ in range(T)]
        for f, (feat, x, ln) in enumerate(zip(wl.features, ids, lengths)):
            t = feat.table
            d = wl.dims[t]
            lid = np.searchsorted(touched[t], x)
            c = int(cols[f])
            gf = grad[:, c: c + d].astype(np.float64)
            got = out[:, c: c + d]
            if feat.pooling == "none":
                assert np.array_equal(got, snap.w[t][lid]), f"{name} feature {f}: gathered rows"
                r, v = O.per_id_grads(lid, None, gf, "none", "exclude")
                _, va = O.per_id_grads(lid, None, np.abs(gf), "none", "exclude")
            else:
                ref, _ = O.pool(snap.w[t], lid, ln, feat.pooling, "exclude")
                mag, _ = O.pool(np.abs(snap.w[t]), lid, ln, feat.pooling, "exclude")
                assert_close(got, ref, rtol, 1e-7, mag, f"{name} feature {f} pooled")
                r, v = O.per_id_grads(lid, ln, gf, feat.pooling, "exclude")
                _, va = O.per_id_grads(lid, ln, np.abs(gf), feat.pooling, "exclude")
            rows_t[t].append(r)
            vals_t[t].append(v)
            absv_t[t].append(va)
        say(name, "outputs checked", f"{time.time() - t0:.1f}s")
        for t in range(T):
            rr, g = O.coalesce(np.concatenate(rows_t[t]), np.concatenate(vals_t[t]))
            _, s = O.coalesce(np.concatenate(rows_t[t]), np.concatenate(absv_t[t]))
            _check_update(f"{name} table {t}", w_post[t], a_post[t], snap.w[t], snap.a[t], rr, g, s, wl.lr, wl.eps,
                          rtol, 1e-7 if wl.dtype == "fp32" else 1e-6, wl.dtype == "bf16")
        say(name, "updates checked", f"{time.time() - t0:.1f}s")
        snap.restore_and_check(dev.tables, dev.states)
        say(name, "untouched rows checked", f"{time.time() - t0:.1f}s")
        STATS.report(name)
    finally:
        del dev
        _free()


def test_sequence_config_full_size_matches_oracle(device):
    """c2: four right-aligned windows of up to 2000 ids over 2e8-row tables
    (10% repeated ids inside a sequence), padded to 2048."""

    t0 = time.time()
    wl = bench.WORKLOADS["c2"]()
    say("c2", "drawing batch")
    rng = np.random.default_rng(1002)
    ids, lengths = bench.draw_batch(rng, wl)
    dev = bench.SequenceDeviceStep(wl, [(ids, lengths)], device)
    try:
        _random_state(dev.states, 6)
        touched = [_touched([m]) for m in ids]
        snap = _Snapshot(dev.tables, dev.states, touched, device)
        torch.cuda.synchronize()
        say("c2", "tables ready", f"{time.time() - t0:.1f}s")
        dev.step(0)
        torch.cuda.synchronize()
        assert int(dev.err.item()) == 0
        say("c2", "step done", f"{time.time() - t0:.1f}s")
        w_post, a_post = snap.after(dev.tables, dev.states)
        _, _, pad = wl.seq_len
        for f, (m, ln) in enumerate(zip(ids, lengths)):
            lid = np.searchsorted(touched[f], m)
            ref, rmask = O.sequence_window(snap.w[f], lid, ln, pad)
            assert np.array_equal(dev.masks[f].cpu().numpy(), rmask), f"c2 feature {f}: mask"
            assert np.array_equal(dev.outs[f].float().cpu().numpy(), ref), f"c2 feature {f}: window"
            del ref
            gf = dev.grads[f].float().cpu().numpy()
            r, v = O.sequence_grads(lid, ln, gf, pad)
            rr, g = O.coalesce(r, v)
            _, s = O.coalesce(r, np.abs(v))
            del gf, v
            _check_update(f"c2 table {f}", w_post[f], a_post[f], snap.w[f], snap.a[f], rr, g, s, wl.lr, wl.eps,
                          RTOL[wl.dtype], 1e-7, False)
            say("c2", f"feature {f} checked", f"{time.time() - t0:.1f}s")
        snap.restore_and_check(dev.tables, dev.states)
        say("c2", "untouched rows checked", f"{time.time() - t0:.1f}s")
        STATS.report("c2")
    finally:
        del dev
        _free()
