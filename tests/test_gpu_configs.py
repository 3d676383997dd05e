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

import gc
import sys
import time

import numpy as np
import pytest
import torch

import bench
from oracle import oracle as O

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(900)]

RTOL = {"fp32": 1e-5, "bf16": 1e-2}


def say(*parts):
    print("CASE", *parts, flush=True)
    sys.stdout.flush()
    sys.stderr.write(" ".join(str(p) for p in ("CASE",) + parts) + "\n")
    sys.stderr.flush()


def _checksum(t: torch.Tensor) -> tuple[int, int]:
    """(sum, sum of squares) of the table's raw bit patterns, as int64 with
    wrap-around; any change to any element changes it but for collisions."""

    x = t.reshape(-1).view(torch.int32 if t.element_size() == 4 else torch.int16)
    s1 = torch.zeros((), dtype=torch.int64, device=t.device)
    s2 = torch.zeros((), dtype=torch.int64, device=t.device)
    step = 1 << 27
    for i in range(0, x.numel(), step):
        part = x[i: i + step].to(torch.int64)
        s1 += part.sum()
        s2 += (part * part).sum()
        del part
    return int(s1.item()), int(s2.item())


def assert_close(got, ref, rtol, atol, scale=None, what=""):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    err = np.abs(got - ref)
    mag = np.abs(ref) if scale is None else np.maximum(np.abs(ref), np.asarray(scale, dtype=np.float64))
    bound = atol + rtol * mag
    bad = err > bound
    assert not bad.any(), f"{what}: {int(bad.sum())} mismatches, worst excess {float((err - bound).max())}"


def _check_update(what, w_post, a_post, w_pre, a_pre, rows, g, s, lr, eps, rtol, atol_w, is_bf16):
    """Touched rows against the oracle's update of the coalesced gradient.

    ``g`` is the oracle's coalesced gradient (fp64) of local ``rows`` and
    ``s`` the same coalesce over |terms|.  fp32 summation puts at most about
    rtol * s on each gradient element, so the accumulator
    a = a0 + sum(g^2)/dim is compared relative to a0 + sum(s^2)/dim, and the
    weight w = w0 - lr * g / (sqrt(a) + eps) relative to |w| plus the
    first-order effect of both errors:
    lr * (s + |g| * a_scale / (2 sqrt(a) (sqrt(a) + eps))) / (sqrt(a) + eps).
    Rows without a gradient must not change at all.
    """

    w_ref, a_ref = O.rowwise_adagrad(w_pre, a_pre, rows, g, lr, eps, is_bf16=is_bf16)
    dim = w_pre.shape[1]
    untouched = np.ones(w_pre.shape[0], dtype=bool)
    untouched[rows] = False
    assert np.array_equal(w_post[untouched], w_pre[untouched]), f"{what}: rows without gradient changed"
    assert np.array_equal(a_post[untouched], a_pre[untouched]), f"{what}: state without gradient changed"
    a_scale = a_pre[rows].astype(np.float64) + (s * s).sum(1) / dim
    assert_close(a_post[rows], a_ref[rows], 1e-5, 1e-7, a_scale, what + " accumulators")
    ar = a_ref[rows].astype(np.float64)
    den = np.sqrt(ar) + eps
    prop = lr * (s + np.abs(g) * (a_scale / (2.0 * np.maximum(np.sqrt(ar), 1e-30) * den))[:, None]) / den[:, None]
    scale = np.abs(w_ref[rows]) + prop
    assert_close(w_post[rows], w_ref[rows], rtol, atol_w, scale, what + " weights")


def _free():
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def _touched(tables_ids):
    return np.unique(np.concatenate([np.zeros(1, np.int64)] + [np.asarray(x, np.int64).ravel() for x in tables_ids]))


class _Snapshot:
    """Touched rows and checksums of every table, taken before the step."""

    def __init__(self, tables, states, touched, device):
        self.idx = [torch.from_numpy(u).to(device) for u in touched]
        self.sums = [(_checksum(w), _checksum(a)) for w, a in zip(tables, states)]
        self.w = [w.index_select(0, i).float().cpu().numpy() for w, i in zip(tables, self.idx)]
        self.a = [a.index_select(0, i).cpu().numpy() for a, i in zip(states, self.idx)]

    def after(self, tables, states):
        w = [t.index_select(0, i).float().cpu().numpy() for t, i in zip(tables, self.idx)]
        a = [s.index_select(0, i).cpu().numpy() for s, i in zip(states, self.idx)]
        return w, a

    def restore_and_check(self, tables, states):
        for t, (w, a, i) in enumerate(zip(tables, states, self.idx)):
            w.index_copy_(0, i, torch.from_numpy(self.w[t]).to(w.device).to(w.dtype))
            a.index_copy_(0, i, torch.from_numpy(self.a[t]).to(a.device))
            assert (_checksum(w), _checksum(a)) == self.sums[t], f"table {t}: an untouched row or state changed"


def _random_state(states, seed):
    gen = torch.Generator(device=states[0].device)
    gen.manual_seed(seed)
    for a in states:
        a.uniform_(0.0, 2.0, generator=gen)


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
    finally:
        del dev
        _free()
