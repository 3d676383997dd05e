"""The mdl_hip torch.library ops on the GPU.

* every op passes ``torch.library.opcheck`` with ROCm tensors;
* the same modules on the CPU and on the GPU, fed the same batches, train to
  the same tables (through the same ops: the CPU and HIP kernels of one schema);
* a ``loss.backward(); optimizer.step()`` loop makes no host synchronisation
  (``torch.cuda.set_sync_debug_mode("error")`` raises on any);
* the grouped row-wise Adagrad and the capacity-padded coalesce against the
  oracle.
"""

import sys

import numpy as np
import pytest
import torch
from torch.library import opcheck

import mdl_amd.library  # noqa: F401
from mdl_amd import ops
from mdl_amd.embeddings import (
    EmbeddingTableSpec,
    ShardedEmbedding,
    grouped_sharded_embedding_lookup,
    plan_embedding_shards,
    pooled_embedding_lookup,
    sequence_embedding_lookup,
)
from mdl_amd.optim import ShardedRowWiseAdagrad
from oracle import oracle as O

pytestmark = pytest.mark.gpu
OPS = torch.ops.mdl_hip


@pytest.fixture
def capacity_grads():
    """Traced backward graphs hold capacity-sized sparse gradients (an exact
    coalesced gradient's size is data); opcheck compares the eager gradient
    with the traced one, so it runs in that mode."""

    mode = mdl_amd.library.sparse_grad_mode()
    mdl_amd.library.set_sparse_grad_mode("capacity")
    yield
    mdl_amd.library.set_sparse_grad_mode(mode)


def announce(*parts):
    print("CASE", *parts, flush=True)
    sys.stdout.flush()


def _to(args, device):
    if isinstance(args, torch.Tensor):
        t = args.to(device)
        if args.requires_grad:
            t = t.detach().requires_grad_(True)
        return t
    if isinstance(args, (list, tuple)):
        return type(args)(_to(a, device) for a in args)
    return args


def test_opcheck_rocm(device, capacity_grads):
    from tests.test_library import _lookup_args

    announce("opcheck_rocm")
    opcheck(OPS.grouped_lookup.default, _to(_lookup_args(), device))
    opcheck(OPS.sequence_lookup.default,
            _to((torch.randn(6, 4, requires_grad=True), torch.tensor([[1, 2, 0], [5, 5, 5]]), torch.tensor([2, 3]), 4,
                 False, 0, True), device))
    opcheck(OPS.rowwise_adagrad_.default,
            _to((torch.randn(10, 4), torch.zeros(10), torch.tensor([1, 3]), torch.randn(2, 4), 0.1, 1e-8), device))
    opcheck(OPS.grouped_rowwise_adagrad_.default,
            _to(([torch.randn(10, 4), torch.randn(5, 8)], [torch.zeros(10), torch.zeros(5)],
                 [torch.tensor([1, 3, 3]), torch.tensor([0])], [torch.randn(3, 4), torch.randn(1, 8)],
                 [torch.tensor([2]), None], [0.1, 0.2], 1e-8), device))
    opcheck(OPS.bucketize.default, _to((torch.tensor([0, -1, 7, -(1 << 63)]), None, 8, "pre_hashed", True), device))
    opcheck(OPS.lengths_to_offsets.default, _to((torch.tensor([3, 0, 2]),), device))
    opcheck(OPS.sparse_coalesce.default, _to((torch.tensor([3, 1, 3]), torch.randn(3, 4), 10), device))
    opcheck(OPS.sparse_coalesce_padded.default, _to((torch.tensor([3, 1, 3]), torch.randn(3, 4), 10), device))


def test_sparse_coalesce_padded_matches_oracle(device):
    announce("sparse_coalesce_padded")
    rng = np.random.default_rng(63)
    idx = (rng.zipf(1.1, size=40000) % 6000).astype(np.int64)
    vals = rng.standard_normal((40000, 24)).astype(np.float32)
    r, v, c = OPS.sparse_coalesce_padded(torch.from_numpy(idx).to(device), torch.from_numpy(vals).to(device), 6000)
    er, ev = O.coalesce(idx, vals.astype(np.float64))
    _, eabs = O.coalesce(idx, np.abs(vals.astype(np.float64)))
    u = int(c.item())
    assert u == er.size and r.numel() == idx.size
    assert np.array_equal(r[:u].cpu().numpy(), er) and bool((r[u:] == er[-1]).all())
    got = v.cpu().numpy()
    assert np.all(np.abs(got[:u] - ev) <= 1e-5 * eabs + 1e-6) and not got[u:].any()


def _modules(specs, device, seed):
    plan = plan_embedding_shards([EmbeddingTableSpec(n, r, d) for n, r, d in specs], world_size=1,
                                 strategy="row_wise", table_wise_max_rows=32)
    torch.manual_seed(seed)
    return [ShardedEmbedding(r, d, table_name=n, shard_spec=plan.tables[n], collect_stats=False).to(device)
            for n, r, d in specs]


def _batches(rng, B, steps):
    out = []
    for _ in range(steps):
        la = rng.integers(0, 9, size=B)
        lb = rng.integers(1, 5, size=B)
        out.append(dict(
            xa=torch.from_numpy(rng.zipf(1.2, size=int(la.sum())) % 300), la=torch.from_numpy(la),
            xb=torch.from_numpy(rng.integers(0, 80, size=int(lb.sum()))), lb=torch.from_numpy(lb),
            xs=torch.from_numpy(rng.integers(0, 500, size=B)),
            seq=torch.from_numpy(rng.integers(0, 500, size=(B, 24))), sl=torch.from_numpy(rng.integers(0, 30, size=B)),
            g=[torch.from_numpy(rng.standard_normal(s).astype(np.float32)) for s in ((B, 8), (B, 4), (B, 16), (B, 16, 16))],
        ))
    return out


def _train(mods, opt, batches, device):
    outs_all = []
    for b in batches:
        opt.zero_grad(set_to_none=True)
        pooled = pooled_embedding_lookup([(mods[0], b["xa"].to(device), b["la"].to(device), "mean", "exclude"),
                                          (mods[1], b["xb"].to(device), b["lb"].to(device), "sum", "exclude")])
        single = grouped_sharded_embedding_lookup([(mods[2], b["xs"].to(device))])[0]
        seq, _ = sequence_embedding_lookup(mods[2], b["seq"].to(device), b["sl"].to(device), target_length=16)
        outs = [pooled[0], pooled[1], single, seq]
        torch.autograd.backward(outs, [g.to(device) for g in b["g"]])
        opt.step()
        outs_all.append([o.detach() for o in outs])
    return outs_all


def test_cpu_and_rocm_modules_train_alike(device):
    """One model on the CPU, one on the GPU, same initial tables and batches:
    outputs, tables and accumulators agree after three steps."""

    announce("cpu_vs_rocm")
    specs = [("bag_a", 300, 8), ("bag_b", 80, 4), ("single", 500, 16)]
    cpu = _modules(specs, "cpu", 3)
    gpu = _modules(specs, device, 3)
    for c, g in zip(cpu, gpu):
        assert torch.equal(c.weight.detach(), g.weight.detach().cpu())
    opt_c = ShardedRowWiseAdagrad([m.weight for m in cpu], lr=0.05, eps=1e-8)
    opt_g = ShardedRowWiseAdagrad([m.weight for m in gpu], lr=0.05, eps=1e-8)
    batches = _batches(np.random.default_rng(7), 48, 3)
    out_c = _train(cpu, opt_c, batches, torch.device("cpu"))
    out_g = _train(gpu, opt_g, batches, device)
    for step, (oc, og) in enumerate(zip(out_c, out_g)):
        for a, b in zip(oc, og):
            torch.testing.assert_close(b.cpu(), a, rtol=1e-5, atol=1e-6, msg=f"step {step} outputs")
    for c, g in zip(cpu, gpu):
        torch.testing.assert_close(g.weight.detach().cpu(), c.weight.detach(), rtol=1e-5, atol=1e-6)
        torch.testing.assert_close(opt_g.state[g.weight]["sum"].cpu(), opt_c.state[c.weight]["sum"], rtol=1e-5,
                                   atol=1e-6)


def test_training_loop_makes_no_host_sync(device, capacity_grads):
    """Lookups (pooled, single, sequence), loss.backward() and
    optimizer.step() under the sync debug mode that raises on any
    device-to-host synchronisation (the capacity-sized gradient mode, which
    reads no row count on the host); the result matches the CPU run."""

    announce("sync_free_loop")
    specs = [("bag_a", 300, 8), ("bag_b", 80, 4), ("single", 500, 16)]
    gpu = _modules(specs, device, 4)
    cpu = _modules(specs, "cpu", 4)
    opt_g = ShardedRowWiseAdagrad([m.weight for m in gpu], lr=0.05, eps=1e-8)
    opt_c = ShardedRowWiseAdagrad([m.weight for m in cpu], lr=0.05, eps=1e-8)
    batches = _batches(np.random.default_rng(8), 64, 3)
    dev_batches = [{k: ([x.to(device) for x in v] if isinstance(v, list) else v.to(device)) for k, v in b.items()}
                   for b in batches]
    # kernels loaded and caches warm before the checked loop
    _train(gpu, opt_g, dev_batches[:1], device)
    _train(cpu, opt_c, batches[:1], torch.device("cpu"))
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        _train(gpu, opt_g, dev_batches[1:], device)
    finally:
        torch.cuda.set_sync_debug_mode("default")
    _train(cpu, opt_c, batches[1:], torch.device("cpu"))
    for c, g in zip(cpu, gpu):
        torch.testing.assert_close(g.weight.detach().cpu(), c.weight.detach(), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_grouped_rowwise_adagrad_matches_oracle(device, dtype):
    """Tables of several dims (wide and unaligned ones too) in one launch,
    each updating only the first ``count`` of its rows."""

    announce("grouped_adagrad", dtype)
    rng = np.random.default_rng(61)
    dims = [16, 24, 7, 300, 64]
    rows = [400, 1000, 50, 120, 3000]
    W = [rng.standard_normal((r, d)).astype(np.float32) for r, d in zip(rows, dims)]
    A = [rng.random(r).astype(np.float32) for r in rows]
    tabs = [torch.from_numpy(w).to(dtype).to(device) for w in W]
    accs = [torch.from_numpy(a).to(device) for a in A]
    caps = [300, 700, 40, 100, 2500]
    present = [123, 700, 0, 57, 2499]
    rr, vv, counts = [], [], []
    for r, c, n, d in zip(rows, caps, present, dims):
        sel = np.sort(rng.choice(r, size=c, replace=False))
        rr.append(torch.from_numpy(sel).to(device))
        vv.append(torch.from_numpy(rng.standard_normal((c, d)).astype(np.float32)).to(dtype).to(device))
        counts.append(torch.tensor([n], device=device))
    counts[1] = None  # all rows
    expect = []
    for t in range(len(rows)):
        n = caps[t] if counts[t] is None else present[t]
        w0 = tabs[t].float().cpu().numpy()
        expect.append(O.rowwise_adagrad(w0, A[t], rr[t][:n].cpu().numpy(), vv[t][:n].float().cpu().numpy(), 0.01 * (t + 1),
                                        1e-8, is_bf16=dtype == torch.bfloat16))
    OPS.grouped_rowwise_adagrad_(tabs, accs, rr, vv, counts, [0.01 * (t + 1) for t in range(len(rows))], 1e-8)
    for t in range(len(rows)):
        wexp, aexp = expect[t]
        np.testing.assert_allclose(accs[t].cpu().numpy(), aexp, rtol=1e-5, atol=1e-7)
        tol = 1e-5 if dtype == torch.float32 else 1e-2
        np.testing.assert_allclose(tabs[t].float().cpu().numpy(), wexp, rtol=tol, atol=1e-6 if tol == 1e-5 else 1e-2)


def test_padded_coalesce_matches_oracle(device):
    """Capacity-sized coalesced gradients: the first count rows are the
    oracle's coalesced rows (bit for bit) and sums; the tail repeats the last
    row with zero values."""

    announce("padded_coalesce")
    rng = np.random.default_rng(62)
    rows, dims = [5000, 40, 700], [32, 16, 12]
    tabs = [torch.zeros((r, d), device=device) for r, d in zip(rows, dims)]
    plan = ops.GroupPlan()
    plan.add_feature(tabs[0], pooling="mean", null_policy="exclude")
    plan.add_feature(tabs[1], pooling="none")
    plan.add_feature(tabs[2], pooling="sum", null_policy="exclude")
    B = 256
    la = rng.integers(0, 20, size=B)
    lc = rng.integers(0, 3, size=B)
    xa = rng.zipf(1.1, size=int(la.sum())) % rows[0]
    xb = rng.integers(0, rows[1], size=B)
    xc = np.zeros(int(lc.sum()), dtype=np.int64)  # all padding: table 2 has no rows
    res = ops.grouped_forward(plan, [torch.from_numpy(x).to(device) for x in (xa, xb, xc)],
                              [torch.from_numpy(la).to(device), None, torch.from_numpy(lc).to(device)],
                              with_backward=True)
    grads = [torch.from_numpy(rng.standard_normal((B, d)).astype(np.float32)).to(device) for d in dims]
    rows_all, vbuf, counts, layout = ops.backward_coalesce_padded(res, grads)
    r, v = ops.split_coalesced(tabs, rows_all, vbuf, layout)
    counts = counts.cpu().numpy()
    for t, (x, ln, mode) in enumerate(((xa, la, "mean"), (xb, None, "none"), (xc, lc, "sum"))):
        ri, vi = O.per_id_grads(x, ln, grads[t].double().cpu().numpy(), mode, "exclude")
        er, ev = O.coalesce(ri, vi)
        u = int(counts[t])
        assert u == er.size and r[t].numel() == x.size
        got_r = r[t].cpu().numpy()
        assert np.array_equal(got_r[:u], er)
        assert np.all(got_r[u:] == (er[-1] if u else 0))
        got_v = v[t].cpu().numpy()
        np.testing.assert_allclose(got_v[:u], ev, rtol=1e-5, atol=1e-5)
        assert not got_v[u:].any()


@pytest.mark.parametrize("grad_mode", ["coalesced", "capacity"])
def test_public_lookup_backward_leaves_its_outputs_alone(device, grad_mode):
    """The grouped_lookup op returns its sort keys and payloads; the backward
    registered on it sorts copies, so the tensors a caller holds keep the
    forward's values (the modules' own node, whose keys nobody else sees,
    sorts in place)."""

    prev = mdl_amd.library.sparse_grad_mode()
    mdl_amd.library.set_sparse_grad_mode(grad_mode)
    try:
        torch.manual_seed(4)
        W = [torch.randn(50, 8, device=device, requires_grad=True), torch.randn(40, 4, device=device,
                                                                                requires_grad=True)]
        ids = [torch.randint(0, 50, (30,), device=device), torch.randint(0, 40, (12,), device=device)]
        lengths = [torch.tensor([3, 0, 9, 18], device=device), None]
        outs, keys, payload, bag_count, offsets, err = OPS.grouped_lookup(W, ids, lengths, [0, 1], [2, 0], [1, 0],
                                                                          [0, 0], True)
        held = (keys.clone(), payload.clone())
        torch.autograd.backward(outs, [torch.randn_like(o) for o in outs])
        assert torch.equal(keys, held[0]) and torch.equal(payload, held[1])
        assert all(w.grad is not None for w in W)
    finally:
        mdl_amd.library.set_sparse_grad_mode(prev)
