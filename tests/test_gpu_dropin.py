"""The drop-in modules on the GPU, written like the reference's own tests
(tests/test_rowwise_adagrad.py, tests/test_sharded_embedding.py:755-802) and
checked against the CPU oracle."""

import json
import pathlib
import sys

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from torch import nn

from mdl_amd.embeddings import (
    EmbeddingTableSpec,
    ShardedEmbedding,
    grouped_sharded_embedding_lookup,
    plan_embedding_shards,
    pooled_embedding_lookup,
)
from mdl_amd.optim import ShardedRowWiseAdagrad
from oracle import oracle as O
from parity_helpers import _check_update

pytestmark = pytest.mark.gpu
GOLD = json.loads((pathlib.Path(__file__).parent / "golden" / "reference_vectors.json").read_text())


def announce(*parts):
    print("CASE", *parts, flush=True)
    sys.stdout.flush()


def _coo(rows, values, size, dtype=torch.float32, device="cuda"):
    idx = torch.tensor([rows], dtype=torch.int64, device=device)
    return torch.sparse_coo_tensor(idx, torch.tensor(values, dtype=dtype, device=device), size=size)


def _modules(device, specs):
    plan = plan_embedding_shards(
        [EmbeddingTableSpec(n, r, d) for n, r, d in specs], world_size=1, strategy="row_wise",
        table_wise_max_rows=32,
    )
    out = []
    for n, r, d in specs:
        m = ShardedEmbedding(r, d, table_name=n, shard_spec=plan.tables[n], padding_idx=0, collect_stats=False)
        out.append(m.to(device))
    return out


@pytest.fixture(params=["coalesced", "capacity"])
def grad_mode(request):
    """Both sparse-gradient modes of the lookups' backward."""

    import mdl_amd.library as L

    mode = L.sparse_grad_mode()
    L.set_sparse_grad_mode(request.param)
    yield request.param
    L.set_sparse_grad_mode(mode)


def test_single_rank_grouped_lookup_matches_native_embedding(device, grad_mode):
    announce("grouped_lookup_native", grad_mode)
    emb_a, emb_b = _modules(device, [("a", 16, 4), ("b", 16, 4)])
    full_a = torch.randn(16, 4)
    full_b = torch.randn(16, 4)
    full_a[0].zero_()
    full_b[0].zero_()
    emb_a.load_full_weight_(full_a.to(device))
    emb_b.load_full_weight_(full_b.to(device))
    ids_a = torch.tensor([0, 3, 3, 7], dtype=torch.long, device=device)
    ids_b = torch.tensor([1, 2, 0, 15], dtype=torch.long, device=device)
    actual = grouped_sharded_embedding_lookup(((emb_a, ids_a), (emb_b, ids_b)))
    torch.testing.assert_close(actual[0].cpu(), F.embedding(ids_a.cpu(), full_a, padding_idx=0))
    torch.testing.assert_close(actual[1].cpu(), F.embedding(ids_b.cpu(), full_b, padding_idx=0))
    loss = actual[0].square().sum() + actual[1].square().sum()
    loss.backward()
    ga = emb_a.weight.grad
    assert ga is not None and ga.is_sparse
    if grad_mode == "coalesced":
        # exact and flagged: the trainer's coalesce() returns the same tensor
        assert ga.is_coalesced() and ga.coalesce() is ga
        assert ga._indices()[0].tolist() == [3, 7]  # padding row 0 gets no gradient
    else:
        # capacity-sized (4 ids): the coalesced rows first, then zero-valued
        # repeats of the last row; the optimizer finds its device row count
        from mdl_amd.library import capacity_grad

        rows, values, count = capacity_grad(emb_a.weight, ga)
        assert int(count.item()) == 2 and ga._indices().size(1) == 4
        assert rows[:2].tolist() == [3, 7]  # padding row 0 gets no gradient
        assert rows[2:].tolist() == [7, 7] and not values[2:].any()
    c = ga.coalesce()
    assert c.indices()[0].tolist() == [3, 7]
    torch.testing.assert_close(c.values().cpu(), torch.stack([4 * full_a[3], 2 * full_a[7]]))
    assert emb_b.weight.grad is not None


def test_out_of_range_ids_raise_index_error(device):
    announce("index_error")
    from mdl_amd.embeddings import index_check_mode, set_index_check_mode

    (emb,) = _modules(device, [("t", 10, 8)])
    # the default check is a device-side assert (like the reference on GPU);
    # a test must not trap the device, so the host-read mode raises here
    assert index_check_mode() == "async"
    set_index_check_mode("sync")
    try:
        with pytest.raises(IndexError, match=r"embedding 't' received IDs outside \[0, 10\): \[10, -1\]"):
            emb(torch.tensor([1, 10, -1], device=device))
    finally:
        set_index_check_mode("async")
    with pytest.raises(TypeError, match="torch.long"):
        emb(torch.tensor([1, 2], dtype=torch.int32, device=device))


def test_adagrad_golden_mean_not_sum(device):
    announce("adagrad_golden_mean_not_sum")
    g = GOLD["rowwise_adagrad_mean_not_sum"]
    p = nn.Parameter(torch.zeros(*g["shape"], device=device))
    opt = ShardedRowWiseAdagrad([p], lr=g["lr"], initial_accumulator_value=0.0, eps=g["eps"])
    p.grad = _coo(g["rows"], g["values"], p.shape, device=device).coalesce()
    opt.step()
    state = opt.state[p]["sum"].cpu()
    for r, a in g["expected_acc"].items():
        assert abs(float(state[int(r)]) - a) < 1e-6
    for r, w in g["expected_neg_weight"].items():
        assert torch.allclose(p[int(r)].neg().cpu(), torch.tensor(w), atol=g["atol"])


def test_adagrad_golden_duplicates_coalesce_once(device):
    announce("adagrad_golden_duplicates")
    g = GOLD["rowwise_adagrad_duplicates_coalesce"]
    p = nn.Parameter(torch.zeros(*g["shape"], device=device))
    opt = ShardedRowWiseAdagrad([p], lr=g["lr"], initial_accumulator_value=0.0, eps=g["eps"])
    p.grad = _coo(g["rows"], g["values"], p.shape, device=device)  # uncoalesced
    opt.step()
    state = opt.state[p]["sum"].cpu()
    assert abs(float(state[3]) - g["expected_acc"]["3"]) < 1e-6
    assert int((state != 0).sum()) == g["expected_nonzero_acc_rows"]


def test_adagrad_golden_empty_gradient_is_noop(device):
    announce("adagrad_golden_empty")
    g = GOLD["rowwise_adagrad_empty_noop"]
    p = nn.Parameter(torch.ones(*g["shape"], device=device))
    opt = ShardedRowWiseAdagrad([p], lr=g["lr"], initial_accumulator_value=g["acc0"])
    before_w = p.detach().clone()
    before_s = opt.state[p]["sum"].clone()
    p.grad = torch.sparse_coo_tensor(torch.empty((1, 0), dtype=torch.int64, device=device),
                                     torch.empty((0, 2), device=device), size=p.shape)
    opt.step()
    assert torch.equal(p, before_w) and torch.equal(opt.state[p]["sum"], before_s)
    assert float(opt.state[p]["step"].item()) == g["expected_step"]


def test_adagrad_golden_bf16_untouched_rows(device):
    announce("adagrad_golden_bf16")
    g = GOLD["rowwise_adagrad_bf16_untouched"]
    p = nn.Parameter(torch.tensor(g["weight"], dtype=torch.bfloat16, device=device))
    before = p.detach().clone()
    opt = ShardedRowWiseAdagrad([p], lr=g["lr"], initial_accumulator_value=0.0, eps=g["eps"])
    p.grad = _coo(g["rows"], g["values"], p.shape, dtype=torch.bfloat16, device=device).coalesce()
    opt.step()
    for r in g["untouched_rows"]:
        assert torch.equal(p[r], before[r])
    assert not torch.equal(p[1], before[1])
    st = opt.state[p]
    assert st["sum"].dtype == torch.float32 and st["step"].device.type == "cpu"
    assert abs(float(st["sum"][1]) - g["expected_acc_row1"]) < 1e-6


def test_state_dict_round_trip_keeps_fp32_accumulator(device):
    announce("state_dict_round_trip")
    p = nn.Parameter(torch.zeros(4, 2, dtype=torch.bfloat16, device=device))
    opt = ShardedRowWiseAdagrad([p], lr=0.1, initial_accumulator_value=0.1)
    p.grad = _coo([0, 2], [[1.0, 2.0], [0.5, 0.5]], p.shape, dtype=torch.bfloat16, device=device).coalesce()
    opt.step()
    q = nn.Parameter(p.detach().clone())
    restored = ShardedRowWiseAdagrad([q], lr=0.1, initial_accumulator_value=0.1)
    restored.load_state_dict(opt.state_dict())
    st = restored.state[q]
    assert st["sum"].dtype == torch.float32 and st["step"].device.type == "cpu"
    assert torch.allclose(st["sum"], opt.state[p]["sum"])
    q.grad = _coo([1], [[1.0, 0.0]], q.shape, dtype=torch.bfloat16, device=device).coalesce()
    restored.step()
    assert st["sum"].dtype == torch.float32


def test_aliased_requests_merge_into_one_update(device):
    """One table in several requests of one grouped call, and in a pooled and
    a direct lookup of the same step (the reference's grouped alias worker,
    tests/test_sharded_embedding.py:198-258, at world size 1): the outputs are
    F.embedding's, and the table gets one row-wise Adagrad update with the sum
    of every request's gradient."""

    announce("aliased_requests")
    user, item = _modules(device, [("user", 13, 4), ("item", 19, 4)])
    full = [torch.arange(13 * 4, dtype=torch.float32).view(13, 4) / 10.0,
            torch.arange(19 * 4, dtype=torch.float32).view(19, 4) / 11.0]
    for m, w in zip((user, item), full):
        w[0].zero_()
        m.load_full_weight_(w.to(device))
    user_ids = torch.tensor([1, 1, 4, 0])
    item_ids = torch.tensor([2, 8, 8])
    repeated_user_ids = torch.tensor([4, 7])
    bag_ids = torch.tensor([7, 0, 3, 3, 12])
    bag_lengths = torch.tensor([2, 0, 3])
    opt = ShardedRowWiseAdagrad([user.weight, item.weight], lr=0.15, eps=1e-8)
    actual = grouped_sharded_embedding_lookup(
        [(user, user_ids.to(device)), (item, item_ids.to(device)), (user, repeated_user_ids.to(device))]
    )
    pooled = pooled_embedding_lookup([(user, bag_ids.to(device), bag_lengths.to(device), "mean", "exclude")])[0]
    expected = [F.embedding(user_ids, full[0], padding_idx=0), F.embedding(item_ids, full[1], padding_idx=0),
                F.embedding(repeated_user_ids, full[0], padding_idx=0)]
    for a, e in zip(actual, expected):
        torch.testing.assert_close(a.cpu(), e)
    loss = sum(o.square().sum() for o in actual) + pooled.square().sum()
    loss.backward()
    opt.step()

    def grads(ids, lengths, out, mode):
        return O.per_id_grads(ids.numpy(), None if lengths is None else lengths.numpy(),
                              2.0 * out.detach().double().cpu().numpy(), mode, "exclude")

    parts = {0: [grads(user_ids, None, actual[0], "none"), grads(repeated_user_ids, None, actual[2], "none"),
                 grads(bag_ids, bag_lengths, pooled, "mean")],
             1: [grads(item_ids, None, actual[1], "none")]}
    for t, m in enumerate((user, item)):
        rows = np.concatenate([r for r, _ in parts[t]])
        vals = np.concatenate([v for _, v in parts[t]])
        r, v = O.coalesce(rows, vals)
        w_ref, a_ref = O.rowwise_adagrad(full[t].numpy(), np.zeros(full[t].shape[0], np.float32), r, v, 0.15, 1e-8)
        got = m.weight.detach().cpu().numpy()
        assert np.allclose(got, w_ref, rtol=1e-5, atol=1e-6), t
        assert np.allclose(opt.state[m.weight]["sum"].cpu().numpy(), a_ref, rtol=1e-5, atol=1e-7), t


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_training_steps_match_oracle(device, dtype):
    """Lookups + mean/sum pooling + loss.backward() + optimizer.step(), 3 steps."""

    announce("training_steps", dtype)
    _train_and_check(device, dtype, [("bag_a", 2000, 32), ("bag_b", 500, 16), ("single", 3000, 64)], seed=90)


@pytest.mark.parametrize("dtype,dims", [(torch.float32, (600, 66, 1030)), (torch.bfloat16, (600, 100, 72))])
def test_wide_rows_train_like_the_reference(device, dtype, dims):
    """Tables of any width train, as with the reference's F.embedding and
    Triton update: rows wider than 64 lanes cover, aligned or not (fp32 600,
    1030 and 66, bf16 600 and 100)."""

    announce("training_steps_wide", dtype, dims)
    _train_and_check(device, dtype, [("bag_a", 2000, dims[0]), ("bag_b", 500, dims[1]), ("single", 3000, dims[2])],
                     seed=91)


def _train_and_check(device, dtype, specs, seed):
    rng = np.random.default_rng(seed)
    mods = _modules(device, specs)
    for m in mods:
        with torch.no_grad():
            w = torch.from_numpy(rng.standard_normal(tuple(m.weight.shape)).astype(np.float32))
            w[0] = 0
            m.weight.data = w.to(dtype).to(device)
    opt = ShardedRowWiseAdagrad([m.weight for m in mods], lr=0.05, eps=1e-8)
    # fp32: 1e-5 relative; bf16 storage: 1e-2 relative.  A bf16 table's
    # sparse gradient is stored in bf16, as the reference's is, so the oracle
    # rounds its coalesced gradient to bf16 before the fp32 update too (else a
    # weight that the step moves across zero differs by that rounding times
    # the step, not by a fraction of itself).  Each step is checked from the
    # tables and accumulators it started from: a one-unit bf16 rounding
    # difference of one step then cannot grow over the next ones.
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    B = 128
    for step in range(3):
        W = [m.weight.detach().float().cpu().numpy().copy() for m in mods]
        A = [opt.state[m.weight]["sum"].cpu().numpy().copy() for m in mods]
        la = rng.integers(0, 12, size=B)
        lb = rng.integers(1, 5, size=B)
        xa = rng.zipf(1.2, size=int(la.sum())) % specs[0][1]
        xb = rng.integers(0, specs[1][1], size=int(lb.sum()))
        xs = rng.integers(0, specs[2][1], size=B)
        opt.zero_grad(set_to_none=True)
        pooled = pooled_embedding_lookup([
            (mods[0], torch.from_numpy(xa).to(device), torch.from_numpy(la).to(device), "mean", "exclude"),
            (mods[1], torch.from_numpy(xb).to(device), torch.from_numpy(lb).to(device), "sum", "exclude"),
        ])
        single = mods[2](torch.from_numpy(xs).to(device))
        outs = [pooled[0], pooled[1], single]
        grads = [torch.from_numpy(rng.standard_normal(tuple(o.shape)).astype(np.float32)).to(dtype).to(device)
                 for o in outs]
        torch.autograd.backward(outs, grads)
        opt.step()
        # oracle
        ra, va = O.per_id_grads(xa, la, grads[0].float().cpu().numpy(), "mean", "exclude")
        rb, vb = O.per_id_grads(xb, lb, grads[1].float().cpu().numpy(), "sum", "exclude")
        rs, vs = O.per_id_grads(xs, None, grads[2].float().cpu().numpy(), "none", "exclude")
        for t, (r, v) in enumerate(((ra, va), (rb, vb), (rs, vs))):
            r, v = O.coalesce(r, v)
            if dtype == torch.bfloat16:
                v = torch.from_numpy(v).to(torch.bfloat16).double().numpy()
            w_ref, a_ref = O.rowwise_adagrad(W[t], A[t], r, v, 0.05, 1e-8, is_bf16=dtype == torch.bfloat16)
            got = mods[t].weight.detach().float().cpu().numpy()
            assert np.all(np.abs(got - w_ref) <= tol * np.abs(w_ref) + tol * 1e-1), (step, t)
            st = opt.state[mods[t].weight]["sum"].cpu().numpy()
            assert np.all(np.abs(st - a_ref) <= tol * np.abs(a_ref) + 1e-6), (step, t)


@pytest.mark.parametrize("order", ["oldest_to_newest", "newest_to_oldest"])
def test_sequence_lookup_forward_backward_step(device, order):
    """sequence_embedding_lookup == F.embedding + right alignment; its sparse
    gradient and the optimizer step match the oracle."""

    from mdl_amd.embeddings import sequence_embedding_lookup

    announce("sequence_lookup", order)
    rng = np.random.default_rng(95)
    (m,) = _modules(device, [("hist", 5000, 32)])
    with torch.no_grad():
        w = torch.from_numpy(rng.standard_normal((5000, 32)).astype(np.float32))
        w[0] = 0
        m.weight.data = w.to(device)
    W0 = m.weight.detach().cpu().numpy().copy()
    opt = ShardedRowWiseAdagrad([m.weight], lr=0.05, eps=1e-8)
    B, L = 40, 300
    lengths = rng.integers(0, L + 1, size=B)
    ids = np.zeros((B, L), dtype=np.int64)
    for b in range(B):
        ids[b, : lengths[b]] = rng.zipf(1.1, size=lengths[b]) % 5000
    for T in (L, 200):
        out, mask = sequence_embedding_lookup(m, torch.from_numpy(ids).to(device),
                                              torch.from_numpy(lengths).to(device), target_length=T,
                                              sequence_order=order)
        ref, rmask = O.sequence_gather(m.weight.detach().cpu().numpy(), ids, lengths, T, order)
        assert np.array_equal(mask.cpu().numpy(), rmask)
        assert np.array_equal(out.detach().cpu().numpy(), ref.astype(np.float32))
    g = rng.standard_normal(tuple(out.shape)).astype(np.float32)
    opt.zero_grad(set_to_none=True)
    out.backward(torch.from_numpy(g).to(device))
    opt.step()
    # oracle: every valid position (b, k) sends grad[b, p(k)] to row ids[b, k]
    rows, vals = [], []
    for b in range(B):
        n = min(int(lengths[b]), T)
        start = T - n
        for k in range(n):
            p = start + k if order == "oldest_to_newest" else start + (n - 1 - k)
            if ids[b, k] != 0:
                rows.append(ids[b, k])
                vals.append(g[b, p])
    rr, vv = O.coalesce(np.array(rows), np.array(vals, dtype=np.float64))
    wexp, aexp = O.rowwise_adagrad(W0, np.zeros(5000, np.float32), rr, vv, 0.05, 1e-8)
    got = m.weight.detach().cpu().numpy()
    _, vabs = O.coalesce(np.array(rows), np.abs(np.array(vals, dtype=np.float64)))
    assert np.all(np.abs(got - wexp) <= 1e-5 * np.abs(wexp) + 1e-6)
    s = opt.state[m.weight]["sum"].cpu().numpy()
    assert np.all(np.abs(s - aexp) <= 1e-5 * np.abs(aexp) + 1e-6)


def test_fused_rowwise_adagrad_update_public_function(device):
    """``fused_rowwise_adagrad_update`` as the reference calls it
    (src/optim.py:68-108): the golden case of tests/test_rowwise_adagrad.py:40-62
    through the function itself, bf16 values on fp32 weights (upcast, as the
    reference does), bf16 weights, and no rows as a no-op."""

    from mdl_amd.optim import fused_rowwise_adagrad_update

    announce("fused_rowwise_adagrad_update")
    g = GOLD["rowwise_adagrad_mean_not_sum"]
    for vdtype in (torch.float32, torch.bfloat16):
        p = torch.zeros(*g["shape"], device=device)
        acc = torch.zeros(g["shape"][0], device=device)
        rows = torch.tensor(g["rows"], device=device)
        fused_rowwise_adagrad_update(p, acc, rows, torch.tensor(g["values"], dtype=vdtype, device=device),
                                     lr=g["lr"], eps=g["eps"])
        for r, a in g["expected_acc"].items():
            assert abs(float(acc[int(r)]) - a) < 1e-6
        for r, w in g["expected_neg_weight"].items():
            assert torch.allclose(p[int(r)].neg().cpu(), torch.tensor(w), atol=g["atol"])
    pb = torch.zeros(*g["shape"], dtype=torch.bfloat16, device=device)
    acc = torch.zeros(g["shape"][0], device=device)
    fused_rowwise_adagrad_update(pb, acc, torch.tensor(g["rows"], device=device),
                                 torch.tensor(g["values"], device=device), lr=g["lr"], eps=g["eps"])
    for r, w in g["expected_neg_weight"].items():  # one rounding to bf16
        assert torch.equal(pb[int(r)].neg().cpu(), torch.tensor(w).to(torch.bfloat16))
    before = pb.clone()
    fused_rowwise_adagrad_update(pb, acc, torch.empty(0, dtype=torch.int64, device=device),
                                 torch.empty((0, 2), device=device), lr=1.0, eps=1e-8)
    assert torch.equal(pb, before)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_concatenated_outputs_train_like_separate_ones(device, dtype):
    """A model that concatenates the lookups into its token slots
    (src/model.py:4395-4420) hands each feature's backward a column slice of
    one [B, sum(D)] gradient.  The slices are read in place and the step
    leaves every weight and accumulator bit-identical to the same gradients
    given as separate contiguous tensors."""

    announce("concatenated_outputs", dtype)
    specs = [("p0", 5000, 16), ("p1", 900, 24), ("s0", 20000, 32), ("s1", 70, 8), ("p2", 3000, 12)]
    rng = np.random.default_rng(41)
    B = 512
    ids, lens = {}, {}
    for n, r, _ in specs:
        if n.startswith("p"):
            ln = rng.integers(0, 7, size=B)
            lens[n] = torch.from_numpy(ln).to(device)
            ids[n] = torch.from_numpy(np.minimum(rng.zipf(1.2, size=int(ln.sum())) - 1, r - 1)).to(device)
        else:
            ids[n] = torch.from_numpy(np.minimum(rng.zipf(1.2, size=B) - 1, r - 1)).to(device)
    g_tokens = torch.randn(B, sum(d for _, _, d in specs), generator=torch.Generator().manual_seed(5)).to(dtype)
    results = []
    for concat in (True, False):
        torch.manual_seed(3)
        mods = [m.to(dtype) for m in _modules(device, specs)]
        opt = ShardedRowWiseAdagrad([m.weight for m in mods], lr=0.05, eps=1e-8)
        by_name = {n: m for (n, _, _), m in zip(specs, mods)}
        for _ in range(2):
            opt.zero_grad(set_to_none=True)
            outs = pooled_embedding_lookup(
                [(by_name[n], ids[n], lens[n], "mean" if n != "p2" else "sum", "exclude") for n, _, _ in specs
                 if n.startswith("p")])
            outs += grouped_sharded_embedding_lookup([(by_name[n], ids[n]) for n, _, _ in specs if n.startswith("s")])
            order = [n for n, _, _ in specs if n.startswith("p")] + [n for n, _, _ in specs if n.startswith("s")]
            dims = {n: d for n, _, d in specs}
            cols = np.concatenate([[0], np.cumsum([dims[n] for n in order])[:-1]])
            g = g_tokens[:, : sum(dims.values())].to(device)
            if concat:
                torch.cat(outs, dim=1).backward(g)
            else:
                parts = [g[:, int(c): int(c) + dims[n]].contiguous() for n, c in zip(order, cols)]
                torch.autograd.backward(outs, parts)
            opt.step()
        torch.cuda.synchronize()
        results.append([m.weight.detach().clone() for m in mods] + [opt.state[m.weight]["sum"].clone() for m in mods])
    for a, b in zip(*results):
        assert torch.equal(a, b)


def _reference_clip(parameters, max_norm):
    """The trainer's sparse clip written with torch ops the way
    src/train.py:5730-5826 writes it (_gradient_values: coalesce and store
    back; fp32 vector_norm of each; min(max_norm / (norm + 1e-6), 1);
    _foreach_mul_ of every value tensor), for a test that keeps the
    reference's own clip in the loop.  Returns the pre-clip norm and whether
    every coalesce() returned its input."""

    grads, untouched = [], True
    for p in parameters:
        g = p.grad
        c = g.coalesce()
        untouched = untouched and c is g
        p.grad = c
        grads.append(c._values())
    total = torch.zeros((), dtype=torch.float32, device=grads[0].device)
    for v in grads:
        total.add_(torch.linalg.vector_norm(v.float(), 2.0).square())
    norm = total.sqrt()
    coef = (max_norm / (norm + 1e-6)).clamp(max=1.0)
    for v in grads:
        v.mul_(coef.to(v.dtype))
    return norm, untouched


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_reference_shaped_step_in_both_gradient_modes(device, grad_mode, dtype):
    """backward -> sparse clip -> ShardedRowWiseAdagrad.step, as the
    reference's trainer sequences them (src/train.py:5730-5826,
    src/optim.py:299-377), against the oracle's coalesce + clip + update.

    coalesced mode: the reference's clip as written, whose coalesce() calls
    must return the gradients as they are (no ATen coalesce);
    capacity mode: the ``mdl_amd.clip`` swap, the whole checked step under
    ``torch.cuda.set_sync_debug_mode("error")`` (no host synchronisation)."""

    from mdl_amd.clip import _clip_sparse_grad_norm

    announce("reference_shaped_step", grad_mode, dtype)
    rng = np.random.default_rng(131)
    specs = [("bag", 400, 16), ("single", 900, 8), ("wide", 300, 130)]
    mods = _modules(device, specs)
    for m in mods:
        m.weight.data = m.weight.data.to(dtype)
    opt = ShardedRowWiseAdagrad([m.weight for m in mods], lr=0.05, eps=1e-8)
    B, max_norm = 64, 0.5

    def batch():
        lb = rng.integers(0, 9, size=B)
        return (torch.from_numpy(rng.zipf(1.2, size=int(lb.sum())) % 400).to(device), torch.from_numpy(lb).to(device),
                torch.from_numpy(rng.integers(0, 900, size=B)).to(device),
                torch.from_numpy(rng.integers(0, 300, size=B)).to(device),
                torch.from_numpy(rng.standard_normal((B, 16 + 8 + 130)).astype(np.float32)).to(device, dtype))

    def step(b):
        xb, lb, xs, xw, g = b
        opt.zero_grad(set_to_none=True)
        pooled = pooled_embedding_lookup([(mods[0], xb, lb, "mean", "exclude")])
        singles = grouped_sharded_embedding_lookup([(mods[1], xs), (mods[2], xw)])
        slots = torch.cat([pooled[0], *singles], dim=1)
        slots.backward(g)
        if grad_mode == "coalesced":
            norm, untouched = _reference_clip([m.weight for m in mods], max_norm)
            assert untouched
        else:
            norm = _clip_sparse_grad_norm([], [m.weight for m in mods], max_norm)
        opt.step()
        return norm

    step(batch())  # kernels loaded, caches warm
    torch.cuda.synchronize()
    W0 = [m.weight.detach().float().cpu().numpy() for m in mods]
    A0 = [opt.state[m.weight]["sum"].cpu().numpy() for m in mods]
    b = batch()
    if grad_mode == "capacity":
        torch.cuda.set_sync_debug_mode("error")
    try:
        norm = step(b)
    finally:
        torch.cuda.set_sync_debug_mode("default")
    xb, lb, xs, xw, g = [t.cpu() for t in b]
    g = g.float().numpy().astype(np.float64)
    parts = [O.per_id_grads(xb.numpy(), lb.numpy(), g[:, :16], "mean", "exclude"),
             O.per_id_grads(xs.numpy(), None, g[:, 16:24], "none", "exclude"),
             O.per_id_grads(xw.numpy(), None, g[:, 24:], "none", "exclude")]
    coalesced = [O.coalesce(r, v) for r, v in parts]
    scaled, total, coef = O.clip_grad_norm([v for _, v in coalesced], max_norm)
    bf16 = dtype == torch.bfloat16
    rtol = 1e-2 if bf16 else 1e-5  # bf16: the sparse gradients are stored in the table dtype
    assert abs(float(norm) - total) <= rtol * total + 1e-6
    absparts = [O.coalesce(r, np.abs(v)) for r, v in parts]
    for t, (m, (r, _), v, (_, s), w0, a0) in enumerate(zip(mods, coalesced, scaled, absparts, W0, A0)):
        # the clipped gradient and its |terms| bound, scaled by the coefficient
        _check_update(f"{grad_mode} table {t}", m.weight.detach().float().cpu().numpy(),
                      opt.state[m.weight]["sum"].cpu().numpy(), w0, a0, r, v, s * coef, 0.05, 1e-8, rtol,
                      1e-6 if bf16 else 1e-7, bf16, acc_rtol=rtol)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_clip_gives_the_same_bits_in_both_gradient_modes(device, dtype):
    """``mdl_amd.clip._clip_sparse_grad_norm`` over capacity-sized gradients
    stops at each table's live rows (a device count in the span) and cuts the
    norm's slices by them, so the norm, the clipped gradients and the update
    equal those of exact coalesced gradients bit for bit."""

    import mdl_amd.library as L
    from mdl_amd.clip import _clip_sparse_grad_norm

    announce("clip_both_modes", dtype)
    specs = [("bag", 400, 16), ("single", 900, 8), ("wide", 300, 130)]
    rng = np.random.default_rng(7)
    B = 96
    lb = rng.integers(0, 9, size=B)
    xb = torch.from_numpy(rng.zipf(1.2, size=int(lb.sum())) % 400).to(device)
    xs = torch.from_numpy(rng.integers(0, 900, size=B)).to(device)
    xw = torch.from_numpy(rng.zipf(1.3, size=B) % 300).to(device)
    lb = torch.from_numpy(lb).to(device)
    g = torch.from_numpy(rng.standard_normal((B, 16 + 8 + 130)).astype(np.float32)).to(device, dtype)
    results = {}
    prev = L.sparse_grad_mode()
    try:
        for mode in ("coalesced", "capacity"):
            L.set_sparse_grad_mode(mode)
            torch.manual_seed(3)
            mods = _modules(device, specs)
            for m in mods:
                m.weight.data = m.weight.data.to(dtype)
            opt = ShardedRowWiseAdagrad([m.weight for m in mods], lr=0.05, eps=1e-8)
            pooled = pooled_embedding_lookup([(mods[0], xb, lb, "mean", "exclude")])
            singles = grouped_sharded_embedding_lookup([(mods[1], xs), (mods[2], xw)])
            torch.cat([pooled[0], *singles], dim=1).backward(g)
            for max_norm in (1e9, 0.25):  # no clipping, then clipping
                norm = _clip_sparse_grad_norm([], [m.weight for m in mods], max_norm)
            opt.step()
            results[mode] = (norm.cpu(), [m.weight.detach().cpu() for m in mods],
                             [opt.state[m.weight]["sum"].cpu() for m in mods])
    finally:
        L.set_sparse_grad_mode(prev)
    (n0, w0, a0), (n1, w1, a1) = results["coalesced"], results["capacity"]
    assert torch.equal(n0, n1)
    for x, y in zip(w0 + a0, w1 + a1):
        assert torch.equal(x, y)


def test_packed_and_separate_ids_look_up_the_same(device):
    """Id tensors that lie back to back in one buffer are read in place (no
    concatenation); separate tensors are concatenated.  Both give the same
    outputs and gradients, bit for bit."""

    announce("packed_ids")
    specs = [("a", 500, 16), ("b", 300, 8), ("c", 700, 32)]
    rng = np.random.default_rng(17)
    B = 40
    la = rng.integers(0, 6, size=B)
    n = [int(la.sum()), B, B]
    packed = torch.from_numpy(rng.integers(0, 300, size=sum(n))).to(device)
    parts = torch.split(packed, n)
    results = []
    for ids in (parts, [p.clone() for p in parts]):
        torch.manual_seed(1)
        mods = _modules(device, specs)
        pooled = pooled_embedding_lookup([(mods[0], ids[0], torch.from_numpy(la).to(device), "mean", "exclude")])
        singles = grouped_sharded_embedding_lookup([(mods[1], ids[1]), (mods[2], ids[2])])
        outs = [pooled[0], *singles]
        torch.autograd.backward(outs, [torch.ones_like(o) for o in outs])
        results.append(([o.detach().cpu() for o in outs], [m.weight.grad.coalesce().to_dense().cpu() for m in mods]))
    for x, y in zip(results[0][0] + results[0][1], results[1][0] + results[1][1]):
        assert torch.equal(x, y)


@pytest.mark.parametrize("grad_mode", ["coalesced", "capacity"])
def test_backward_over_a_retained_graph_repeats_its_gradient(device, grad_mode):
    """The modules' backward sorts the forward's keys in place; a second
    backward over the retained graph sorts the sorted pairs again and gives
    the same gradient, so the accumulated one is exactly twice the first."""

    import mdl_amd.library as L

    announce("retained_graph", grad_mode)
    prev = L.sparse_grad_mode()
    L.set_sparse_grad_mode(grad_mode)
    try:
        rng = np.random.default_rng(23)
        mods = _modules(device, [("bag", 300, 16), ("single", 200, 8)])
        B = 64
        lb = rng.integers(0, 7, size=B)
        xb = torch.from_numpy(rng.zipf(1.2, size=int(lb.sum())) % 300).to(device)
        xs = torch.from_numpy(rng.zipf(1.2, size=B) % 200).to(device)
        pooled = pooled_embedding_lookup([(mods[0], xb, torch.from_numpy(lb).to(device), "mean", "exclude")])
        single = grouped_sharded_embedding_lookup([(mods[1], xs)])
        g = [torch.randn(B, 16, device=device), torch.randn(B, 8, device=device)]
        torch.autograd.backward([pooled[0], single[0]], g, retain_graph=True)
        first = [m.weight.grad.coalesce().to_dense().clone() for m in mods]
        torch.autograd.backward([pooled[0], single[0]], g)
        for m, f in zip(mods, first):
            assert torch.equal(m.weight.grad.coalesce().to_dense(), 2 * f)
    finally:
        L.set_sparse_grad_mode(prev)
