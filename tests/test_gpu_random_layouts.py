"""Randomised layouts through the fused step, checked against the oracle.

Each seed draws a whole plan: 2-8 tables of 2 to 200 k rows, widths from 1
to 300 (rows narrower than a lane's vector, unaligned rows, rows wider than
a wave covers), fp32 or bf16 per table, 2-10 features over them (tables
read by several features, pooled by sum or mean under either null policy,
or unpooled), bags of 0-12 ids, Zipf or uniform ids with padding ids and
ids outside their table.  One ``SparseStep`` step (lookup, sort, segment
reduce, row-wise Adagrad) is compared with ``oracle.sparse_step`` on the
outputs, every weight row and every accumulator (src/model.py:509-678,
src/optim.py:31-62,299-357), and the step's error count with the number of
ids outside their table (src/embeddings.py:140-147).  The drop-in modules
and optimizer are then trained under drawn request lists, and
``SequenceStep`` run over drawn sequence layouts, the same way.
"""

import sys
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from mdl_amd import ops
from mdl_amd.sparse_step import SparseStep
from oracle import oracle as O
from parity_helpers import _check_update, assert_close

pytestmark = pytest.mark.gpu

WIDTHS = [1, 2, 3, 4, 8, 12, 16, 24, 32, 48, 64, 100, 128, 130, 256, 300]


def announce(*parts):
    print("CASE", *parts, flush=True)
    sys.stdout.flush()


def _draw(seed):
    rng = np.random.default_rng(1000 + seed)
    T = int(rng.integers(2, 9))
    rows = [int(np.exp(rng.uniform(np.log(2), np.log(200_000)))) for _ in range(T)]
    dims = [int(rng.choice(WIDTHS)) for _ in range(T)]
    bf16 = [bool(rng.random() < 0.4) for _ in range(T)]
    F = int(rng.integers(2, 11))
    feats = []
    for f in range(F):
        t = int(rng.integers(0, T)) if (f >= T or rng.random() < 0.3) else f
        feats.append({"table": t, "pooling": int(rng.choice([0, 1, 2])), "exclude": int(rng.integers(0, 2))})
    return rng, rows, dims, bf16, feats


def _ids(rng, n, rows):
    zipf = rng.random() < 0.5
    x = (rng.zipf(1.2, size=n) - 1) % rows if zipf else rng.integers(0, rows, size=n)
    x = x.astype(np.int64)
    x[rng.random(n) < 0.05] = 0                                # padding / null ids
    bad = rng.random(n) < 0.01
    x[bad] = np.where(rng.random(int(bad.sum())) < 0.5, rows + rng.integers(0, 5, int(bad.sum())), -1)
    return x


def _random_step(device, seed, error_count=None):
    """The drawn layout of ``seed`` as a ``SparseStep`` with its host data."""

    rng, rows, dims, bf16, feats = _draw(seed)
    B = int(rng.integers(1, 700))
    W0 = []
    for r, d, b in zip(rows, dims, bf16):
        w = rng.standard_normal((r, d)).astype(np.float32)
        if b:
            w = torch.from_numpy(w).to(torch.bfloat16).float().numpy()
        W0.append(w)
    A0 = [rng.random(r).astype(np.float32) for r in rows]
    tabs = [torch.from_numpy(w).to(torch.bfloat16 if b else torch.float32).to(device) for w, b in zip(W0, bf16)]
    accs = [torch.from_numpy(a.copy()).to(device) for a in A0]
    plan = ops.GroupPlan()
    for f in feats:
        plan.add_feature(tabs[f["table"]], pooling={0: "none", 1: "sum", 2: "mean"}[f["pooling"]],
                         null_policy="exclude" if f["exclude"] else "include_as_padding", state=accs[f["table"]])
    ids, lens, parts = [], [], []
    for f in feats:
        t = f["table"]
        if f["pooling"] == 0:
            x = _ids(rng, B, rows[t])
            lens.append(None)
            parts.append(np.array([B]))
        else:
            ln = rng.integers(0, 13, size=B)
            ln[rng.random(B) < 0.1] = 0
            x = _ids(rng, int(ln.sum()), rows[t])
            lens.append(ln)
            parts.append(ln)
        ids.append(x)
    fdims = [dims[f["table"]] for f in feats]
    fdt = [torch.bfloat16 if bf16[f["table"]] else torch.float32 for f in feats]
    S = sum(fdims)
    cols = np.concatenate([[0], np.cumsum(fdims)[:-1]]).astype(np.int64)
    g_slot = rng.standard_normal((B, S))
    outs = [torch.empty((B, d), dtype=dt, device=device) for d, dt in zip(fdims, fdt)]
    grads = []
    for f, (c, d, dt) in enumerate(zip(cols, fdims, fdt)):
        g = torch.from_numpy(g_slot[:, c: c + d].astype(np.float32)).to(dt)
        g_slot[:, c: c + d] = g.double().numpy()  # the oracle sees the rounded gradient
        grads.append(g.to(device))
    step = SparseStep(plan, torch.from_numpy(np.concatenate(ids)).to(device),
                      torch.from_numpy(np.concatenate(parts)).to(device), [x.size for x in ids],
                      [0 if ln is None else B for ln in lens], outs, grads, error_count=error_count)
    return SimpleNamespace(step=step, rows=rows, dims=dims, bf16=bf16, feats=feats, B=B, W0=W0, A0=A0, tabs=tabs,
                           accs=accs, ids=ids, lens=lens, fdims=fdims, fdt=fdt, S=S, cols=cols, g_slot=g_slot,
                           outs=outs)


@pytest.mark.parametrize("seed", range(40))
def test_random_layout_step_matches_oracle(device, seed):
    err = torch.zeros(1, dtype=torch.int32, device=device)
    z = _random_step(device, seed, err)
    announce("random_layout", seed, z.rows, z.dims, z.bf16, z.feats, z.B)
    rows, bf16, feats, B, W0, A0, tabs, accs = z.rows, z.bf16, z.feats, z.B, z.W0, z.A0, z.tabs, z.accs
    ids, lens, fdims, fdt, S, cols, g_slot, outs, step = (z.ids, z.lens, z.fdims, z.fdt, z.S, z.cols, z.g_slot,
                                                          z.outs, z.step)
    lr, eps = 0.03, 1e-8
    step.step(lr, eps)
    torch.cuda.synchronize()

    ofeats, offs, bag_off, ids_off = [], [], 0, 0
    for f, x, ln, c in zip(feats, ids, lens, cols):
        ofeats.append({"table": f["table"], "pooling": f["pooling"], "exclude": f["exclude"], "ids_off": ids_off,
                       "bag_off": bag_off, "num_bags": 0 if ln is None else B, "out_col": int(c)})
        if ln is not None:
            o = O.offsets_of(ln)
            offs.append(o)
            bag_off += len(o)
        ids_off += x.size
    off_all = np.concatenate(offs) if offs else np.zeros(1, np.int64)
    tables = [{"W": w.copy(), "acc": a.copy(), "is_bf16": b} for w, a, b in zip(W0, A0, bf16)]
    ref = O.sparse_step(ofeats, tables, np.concatenate(ids), off_all, S, g_slot, lr, eps)
    absw = [{"W": np.abs(w), "acc": np.zeros_like(a)} for w, a in zip(W0, A0)]
    mag = O.sparse_step(ofeats, absw, np.concatenate(ids), off_all, S, np.zeros_like(g_slot), 0.0, 1.0)

    n_bad = sum(int(((x < 0) | (x >= rows[f["table"]])).sum()) for f, x in zip(feats, ids))
    assert int(err.item()) == n_bad
    for f, (o, c, d) in enumerate(zip(outs, cols, fdims)):
        rt = 1e-2 if fdt[f] == torch.bfloat16 else 1e-5
        assert_close(o.float().cpu().numpy(), ref[:, c: c + d], rt, 1e-6 if rt < 1e-3 else 1e-2,
                     mag[:, c: c + d], what=f"output of feature {f}")
    for t in range(len(rows)):
        rt = 1e-2 if bf16[t] else 1e-5
        assert_close(tabs[t].float().cpu().numpy(), tables[t]["W"], rt, 1e-6 if not bf16[t] else 1e-2,
                     what=f"weights of table {t}")
        assert_close(accs[t].cpu().numpy(), tables[t]["acc"], 1e-5, 1e-7, what=f"accumulators of table {t}")


@pytest.mark.parametrize("seed", range(12))
def test_random_dropin_training_matches_oracle(device, seed):
    """The drop-in modules under drawn request lists: 3-7 ``ShardedEmbedding``
    tables (widths 1-300, fp32 or bf16 each), pooled requests (sum or mean,
    either null policy) through ``pooled_embedding_lookup``, unpooled ones
    through ``grouped_sharded_embedding_lookup``, a table requested several
    times in one step (its gradients merge), two ``ShardedRowWiseAdagrad``
    steps.  Each step is checked from the weights and accumulators it began
    with against the oracle, within bounds set by the same sums over |terms|
    (a row whose terms cancel keeps an fp32 error of rtol * sum|terms|):
    per-id gradients of every request
    (src/model.py:564-570), coalesced per table (src/optim.py:321-324), the
    row-wise update (src/optim.py:31-62); a bf16 table's gradient is stored
    in bf16 as the reference's is.  Odd seeds run with capacity-sized
    gradients, even ones with exact coalesced ones; every third seed
    accumulates two backward passes before each step
    (src/train.py:5388-5396), and seeds 1, 5 and 9 clip the gradients
    through ``mdl_amd.clip._clip_sparse_grad_norm`` first (src/train.py:5788-5826)."""

    import mdl_amd.library as L
    from mdl_amd.clip import _clip_sparse_grad_norm
    from mdl_amd.embeddings import (EmbeddingTableSpec, ShardedEmbedding, grouped_sharded_embedding_lookup,
                                    plan_embedding_shards, pooled_embedding_lookup)
    from mdl_amd.optim import ShardedRowWiseAdagrad

    grad_mode = "capacity" if seed % 2 else "coalesced"
    passes = 2 if seed % 3 == 0 else 1
    clip = 0.5 if seed % 4 == 1 else None
    prev_mode = L.sparse_grad_mode()
    L.set_sparse_grad_mode(grad_mode)
    try:
        _random_dropin(device, seed, passes, clip, _clip_sparse_grad_norm, EmbeddingTableSpec, ShardedEmbedding,
                       grouped_sharded_embedding_lookup, plan_embedding_shards, pooled_embedding_lookup,
                       ShardedRowWiseAdagrad)
    finally:
        L.set_sparse_grad_mode(prev_mode)


def _random_dropin(device, seed, passes, clip, _clip_sparse_grad_norm, EmbeddingTableSpec, ShardedEmbedding,
                   grouped_sharded_embedding_lookup, plan_embedding_shards, pooled_embedding_lookup,
                   ShardedRowWiseAdagrad):
    rng = np.random.default_rng(5000 + seed)
    T = int(rng.integers(3, 8))
    rows = [int(np.exp(rng.uniform(np.log(3), np.log(100_000)))) for _ in range(T)]
    dims = [int(rng.choice(WIDTHS)) for _ in range(T)]
    bf16 = [bool(rng.random() < 0.4) for _ in range(T)]
    announce("random_dropin", seed, rows, dims, bf16, passes, clip)
    specs = [(f"t{t}", rows[t], dims[t]) for t in range(T)]
    plan = plan_embedding_shards([EmbeddingTableSpec(n, r, d) for n, r, d in specs], world_size=1,
                                 strategy="row_wise", table_wise_max_rows=32)
    mods = []
    for (n, r, d), b in zip(specs, bf16):
        m = ShardedEmbedding(r, d, table_name=n, shard_spec=plan.tables[n], collect_stats=False,
                             dtype=torch.bfloat16 if b else torch.float32).to(device)
        mods.append(m)
    opt = ShardedRowWiseAdagrad([m.weight for m in mods], lr=0.05, eps=1e-8)
    B = int(rng.integers(1, 300))
    for step in range(2):
        W = [m.weight.detach().float().cpu().numpy().copy() for m in mods]
        A = [opt.state[m.weight]["sum"].cpu().numpy().copy() for m in mods]
        opt.zero_grad(set_to_none=True)
        per_table = {t: ([], [], []) for t in range(T)}
        for _ in range(passes):
            pooled_req, single_req, ref_req = [], [], []
            for _ in range(int(rng.integers(2, 9))):
                t = int(rng.integers(0, T))
                if rng.random() < 0.6:
                    ln = rng.integers(0, 9, size=B)
                    x = np.minimum(rng.zipf(1.2, size=int(ln.sum())) - 1, rows[t] - 1)
                    mode = "mean" if rng.random() < 0.5 else "sum"
                    pol = "exclude" if rng.random() < 0.5 else "include_as_padding"
                    pooled_req.append((mods[t], torch.from_numpy(x).to(device), torch.from_numpy(ln).to(device),
                                       mode, pol))
                    ref_req.append(("p", t, x, ln, mode, pol))
                else:
                    x = rng.integers(0, rows[t], size=B)
                    single_req.append((mods[t], torch.from_numpy(x).to(device)))
                    ref_req.append(("s", t, x, None, "none", "exclude"))
            outs = (pooled_embedding_lookup(pooled_req) if pooled_req else []) + \
                   (grouped_sharded_embedding_lookup(single_req) if single_req else [])
            order = [r for r in ref_req if r[0] == "p"] + [r for r in ref_req if r[0] == "s"]
            grads = [torch.from_numpy(rng.standard_normal(tuple(o.shape)).astype(np.float32)).to(o.dtype).to(device)
                     for o in outs]
            torch.autograd.backward(outs, grads)
            for (kind, t, x, ln, mode, pol), g in zip(order, grads):
                gh = g.float().cpu().numpy()
                r, v = O.per_id_grads(x, ln, gh, mode, pol)
                _, va = O.per_id_grads(x, ln, np.abs(gh), mode, pol)
                per_table[t][0].append(r)
                per_table[t][1].append(v.reshape(-1, dims[t]))
                per_table[t][2].append(va.reshape(-1, dims[t]))
        coalesced = {}
        for t in range(T):
            if per_table[t][0]:
                r, v = O.coalesce(np.concatenate(per_table[t][0]), np.concatenate(per_table[t][1]))
                _, va = O.coalesce(np.concatenate(per_table[t][0]), np.concatenate(per_table[t][2]))
            else:
                r, v, va = np.zeros(0, np.int64), np.zeros((0, dims[t])), np.zeros((0, dims[t]))
            if bf16[t]:
                v = torch.from_numpy(v).to(torch.bfloat16).double().numpy()
            coalesced[t] = (r, v, va)
        coef = 1.0
        if clip is not None:
            norm = _clip_sparse_grad_norm([], [m.weight for m in mods], clip)
            _, total, coef = O.clip_grad_norm([coalesced[t][1] for t in range(T)], clip)
            rt = 1e-2 if any(bf16) else 1e-5
            assert abs(float(norm) - total) <= rt * total + 1e-6, (float(norm), total)
        opt.step()
        for t in range(T):
            r, v, va = coalesced[t]
            # a bf16 table's gradient is rounded to bf16 once per backward
            # pass, and accumulated passes once more when the optimizer
            # coalesces them: up to three roundings of 2^-9 each
            rt = (1e-2 if passes == 1 else 2e-2) if bf16[t] else 1e-5
            _check_update(f"step {step} table {t}", mods[t].weight.detach().float().cpu().numpy(),
                          opt.state[mods[t].weight]["sum"].cpu().numpy(), W[t], A[t], r, v * coef, va * coef,
                          0.05, 1e-8, rt, 1e-6 if bf16[t] else 1e-7, bf16[t], acc_rtol=rt)


@pytest.mark.parametrize("seed", range(12))
def test_random_sequence_step_matches_oracle(device, seed):
    """``SequenceStep`` over drawn sequence layouts: 1-4 features over tables
    of 2 to 100 k rows (one table read by several features, widths 1-300,
    fp32 or bf16 each), input lengths 1-300 and windows 1-300 wide, row
    lengths from 0 to past the input, padding ids, junk ids past each row's
    length (never read), either order.  Windows and masks are compared bit
    for bit with the oracle's gather (src/model.py:2989-3100), and every
    table's update with the oracle's coalesce + row-wise Adagrad of the
    window gradients (src/optim.py:31-62), within bounds from the sums over
    |terms|."""

    from mdl_amd.sparse_step import SequenceStep

    rng = np.random.default_rng(7000 + seed)
    F = int(rng.integers(1, 5))
    T = int(rng.integers(1, F + 1))
    rows = [int(np.exp(rng.uniform(np.log(2), np.log(100_000)))) for _ in range(T)]
    dims = [int(rng.choice(WIDTHS)) for _ in range(T)]
    bf16 = [bool(rng.random() < 0.4) for _ in range(T)]
    table_of = [f if f < T else int(rng.integers(0, T)) for f in range(F)]
    order = "oldest_to_newest" if rng.random() < 0.5 else "newest_to_oldest"
    B = int(rng.integers(1, 200))
    L_in = [int(rng.integers(1, 301)) for _ in range(F)]
    L_out = [int(rng.integers(1, 301)) for _ in range(F)]
    announce("random_sequence", seed, rows, dims, bf16, table_of, order, B, L_in, L_out)
    W0 = []
    for r, d, b in zip(rows, dims, bf16):
        w = rng.standard_normal((r, d)).astype(np.float32)
        W0.append(torch.from_numpy(w).to(torch.bfloat16).float().numpy() if b else w)
    A0 = [rng.random(r).astype(np.float32) for r in rows]
    tabs = [torch.from_numpy(w).to(torch.bfloat16 if b else torch.float32).to(device) for w, b in zip(W0, bf16)]
    accs = [torch.from_numpy(a.copy()).to(device) for a in A0]
    plan = ops.GroupPlan()
    for f in range(F):
        plan.add_feature(tabs[table_of[f]], pooling="none", state=accs[table_of[f]])
    ids, lens, outs, masks, grads = [], [], [], [], []
    for f in range(F):
        t = table_of[f]
        ln = rng.integers(0, L_in[f] + 6, size=B)
        m = rng.integers(-5, rows[t] + 5, size=(B, L_in[f]))  # junk past each row's length
        for b in range(B):
            n = min(int(ln[b]), L_in[f])
            x = (rng.zipf(1.2, size=n) - 1) % rows[t]
            x[rng.random(n) < 0.05] = 0
            m[b, :n] = x
        ids.append(m.astype(np.int64))
        lens.append(ln)
        dt = torch.bfloat16 if bf16[t] else torch.float32
        outs.append(torch.empty((B, L_out[f], dims[t]), dtype=dt, device=device))
        masks.append(torch.empty((B, L_out[f]), dtype=torch.bool, device=device))
        grads.append(torch.from_numpy(rng.standard_normal((B, L_out[f], dims[t])).astype(np.float32)).to(dt)
                     .to(device))
    err = torch.zeros(1, dtype=torch.int32, device=device)
    st = SequenceStep(plan, [torch.from_numpy(m).to(device) for m in ids],
                      [torch.from_numpy(ln).to(device) for ln in lens], outs, masks, grads, order=order,
                      error_count=err)
    lr, eps = 0.03, 1e-8
    st.step(lr, eps)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    per_table = {t: ([], [], []) for t in range(T)}
    for f in range(F):
        t = table_of[f]
        ref, rmask = O.sequence_window(W0[t], ids[f], lens[f], L_out[f], order)
        assert np.array_equal(outs[f].float().cpu().numpy(), ref.astype(np.float32)), f"window of feature {f}"
        assert np.array_equal(masks[f].cpu().numpy(), rmask), f"mask of feature {f}"
        g = grads[f].float().cpu().numpy()
        r, v = O.sequence_grads(ids[f], lens[f], g, L_out[f], order)
        _, va = O.sequence_grads(ids[f], lens[f], np.abs(g), L_out[f], order)
        per_table[t][0].append(r)
        per_table[t][1].append(v.reshape(-1, dims[t]))
        per_table[t][2].append(va.reshape(-1, dims[t]))
    for t in range(T):
        r, v = O.coalesce(np.concatenate(per_table[t][0]), np.concatenate(per_table[t][1]))
        _, va = O.coalesce(np.concatenate(per_table[t][0]), np.concatenate(per_table[t][2]))
        rt = 1e-2 if bf16[t] else 1e-5
        _check_update(f"table {t}", tabs[t].float().cpu().numpy(), accs[t].cpu().numpy(), W0[t], A0[t], r, v, va,
                      lr, eps, rt, 1e-6 if bf16[t] else 1e-7, bf16[t])


@pytest.mark.parametrize("seed", range(8))
def test_random_layout_graph_replays_match_eager(device, seed):
    """A captured step of a drawn layout (every kernel variant the layout
    needs: widths, dtypes, aliased tables, the clip on odd seeds) replays bit
    for bit like eager steps on an identical copy, with eager work and a
    synchronisation between the replays."""

    eager = _random_step(device, seed)
    graph = _random_step(device, seed)
    clip = 1.0 if seed % 2 else None
    announce("random_layout_graph", seed, eager.rows, eager.dims, eager.bf16, eager.feats, eager.B, clip)
    lr, eps = 0.03, 1e-8
    eager.step.step(lr, eps, clip)
    graph.step.step(lr, eps, clip)  # loads the kernels before the recording
    graph.step.capture(lr, eps, clip)
    for r in range(3):
        eager.step.step(lr, eps, clip)
        graph.step.replay()
        torch.cuda.synchronize()
        _ = float(graph.tabs[0].double().sum())  # eager work between replays
        for a, b in zip(graph.outs + graph.tabs + graph.accs, eager.outs + eager.tabs + eager.accs):
            assert torch.equal(a, b), f"replay {r}"
