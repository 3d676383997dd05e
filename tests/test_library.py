"""The mdl_hip torch.library ops on the CPU (no GPU needed).

Every op passes ``torch.library.opcheck`` (schema, autograd registration,
fake tensors, AOT dispatch); the drop-in modules train on CPU parameters
through the same ops, checked against the C oracle and the reference tests'
golden vectors (tests/test_rowwise_adagrad.py); the CPU bucketing matches
the oracle bit for bit.
"""

import json
import pathlib

import numpy as np
import pytest
import torch
from torch import nn
from torch.library import opcheck

import mdl_amd.library  # noqa: F401  (registers the ops)
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

GOLD = json.loads((pathlib.Path(__file__).parent / "golden" / "reference_vectors.json").read_text())
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


def _lookup_args(requires_grad=True):
    torch.manual_seed(0)
    W = [torch.randn(20, 4, requires_grad=requires_grad), torch.randn(9, 8, requires_grad=requires_grad)]
    ids = [torch.tensor([1, 0, 5, 5, 19]), torch.tensor([[3, 4], [0, 8]]), torch.tensor([2, 2, 7])]
    ln = [torch.tensor([2, 0, 3]), None, torch.tensor([1, 2])]
    return (W, ids, ln, [0, 1, 1], [2, 0, 1], [1, 0, 0], [0, 0, 0], True)


@pytest.mark.parametrize("name", ["grouped_lookup", "sequence_lookup", "rowwise_adagrad_", "grouped_rowwise_adagrad_",
                                  "bucketize", "lengths_to_offsets", "sparse_coalesce", "sparse_coalesce_padded",
                                  "grouped_lookup_backward",
                                  "sequence_lookup_backward"])
def test_opcheck_cpu(name, capacity_grads):
    if name == "grouped_lookup":
        args = _lookup_args()
    elif name == "grouped_lookup_backward":
        W, ids, ln, table, pooling, exclude, pad, _ = _lookup_args(False)
        grads = [torch.randn(3, 4), torch.randn(2, 2, 8), torch.randn(2, 8)]
        e = torch.empty(0, dtype=torch.int32)
        args = (W, ids, ln, table, pooling, exclude, pad, grads, e, e.clone(), torch.zeros(8), torch.zeros(0,
                                                                                                        dtype=torch.int64))
    elif name == "sequence_lookup":
        args = (torch.randn(6, 4, requires_grad=True), torch.tensor([[1, 2, 0], [5, 5, 5]]), torch.tensor([2, 3]), 4,
                False, 0, True)
    elif name == "sequence_lookup_backward":
        e = torch.empty(0, dtype=torch.int32)
        args = (torch.randn(6, 4), torch.tensor([[1, 2, 0], [5, 5, 5]]), torch.tensor([2, 3]), 4, True, 0,
                torch.randn(2, 4, 4), e, e.clone())
    elif name == "rowwise_adagrad_":
        args = (torch.randn(10, 4), torch.zeros(10), torch.tensor([1, 3]), torch.randn(2, 4), 0.1, 1e-8)
    elif name == "grouped_rowwise_adagrad_":
        args = ([torch.randn(10, 4), torch.randn(5, 2)], [torch.zeros(10), torch.zeros(5)],
                [torch.tensor([1, 3, 3]), torch.tensor([0])], [torch.randn(3, 4), torch.randn(1, 2)],
                [torch.tensor([2]), None], [0.1, 0.2], 1e-8)
    elif name == "bucketize":
        args = (torch.tensor([0, -1, 7, -(1 << 63)]), torch.tensor([1, 1, 0, 1], dtype=torch.uint8), 8, "pre_hashed",
                True)
    elif name == "lengths_to_offsets":
        args = (torch.tensor([3, 0, 2]),)
    else:
        args = (torch.tensor([3, 1, 3]), torch.randn(3, 4), 10)
    opcheck(getattr(OPS, name).default, args)


def test_cpu_bucketize_matches_oracle_bit_for_bit():
    rng = np.random.default_rng(5)
    raw = rng.integers(-(1 << 63), (1 << 63) - 1, size=20000, dtype=np.int64, endpoint=True)
    raw[:4] = [-(1 << 63), (1 << 63) - 1, 0, -1]
    valid = (rng.random(raw.size) > 0.1).astype(np.uint8)
    for buckets in (1, 8, 1 << 20, 1 << 40):
        out, err = OPS.bucketize(torch.from_numpy(raw), torch.from_numpy(valid), buckets, "pre_hashed", True)
        ref, zeros = O.bucketize_pre_hashed(raw, buckets, valid)
        assert np.array_equal(out.numpy(), ref) and int(err) == zeros
    for rows in (2, 3, 1_000_000, (1 << 40) + 2, (1 << 62) + 1):
        out, _ = OPS.bucketize(torch.from_numpy(raw), None, rows, "mod", False)
        assert np.array_equal(out.numpy(), O.bucketize_mod(raw, rows))


def _modules(specs, dtype=torch.float32):
    plan = plan_embedding_shards([EmbeddingTableSpec(n, r, d) for n, r, d in specs], world_size=1,
                                 strategy="row_wise", table_wise_max_rows=32)
    return [ShardedEmbedding(r, d, table_name=n, shard_spec=plan.tables[n], collect_stats=False, dtype=dtype)
            for n, r, d in specs]


def test_cpu_training_steps_match_oracle():
    """Mean and sum bags plus a single-valued lookup, loss.backward() and
    optimizer.step() on CPU parameters, three steps, against the C oracle."""

    rng = np.random.default_rng(91)
    mods = _modules([("bag_a", 300, 8), ("bag_b", 80, 4), ("single", 500, 16)])
    opt = ShardedRowWiseAdagrad([m.weight for m in mods], lr=0.05, eps=1e-8)
    W = [m.weight.detach().numpy().copy() for m in mods]
    A = [np.zeros(m.weight.shape[0], np.float32) for m in mods]
    B = 64
    for step in range(3):
        la = rng.integers(0, 9, size=B)
        lb = rng.integers(1, 5, size=B)
        xa = rng.zipf(1.2, size=int(la.sum())) % 300
        xb = rng.integers(0, 80, size=int(lb.sum()))
        xs = rng.integers(0, 500, size=B)
        opt.zero_grad(set_to_none=True)
        pooled = pooled_embedding_lookup([(mods[0], torch.from_numpy(xa), torch.from_numpy(la), "mean", "exclude"),
                                          (mods[1], torch.from_numpy(xb), torch.from_numpy(lb), "sum", "exclude")])
        single = grouped_sharded_embedding_lookup([(mods[2], torch.from_numpy(xs))])[0]
        outs = [pooled[0], pooled[1], single]
        grads = [torch.randn(o.shape) for o in outs]
        torch.autograd.backward(outs, grads)
        opt.step()
        for t, (x, ln, mode) in enumerate(((xa, la, "mean"), (xb, lb, "sum"), (xs, None, "none"))):
            r, v = O.per_id_grads(x, ln, grads[t].double().numpy(), mode, "exclude")
            r, v = O.coalesce(r, v)
            W[t], A[t] = O.rowwise_adagrad(W[t], A[t], r, v, 0.05, 1e-8)
    for t, m in enumerate(mods):
        np.testing.assert_allclose(m.weight.detach().numpy(), W[t], rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(opt.state[m.weight]["sum"].numpy(), A[t], rtol=1e-5, atol=1e-6)
        assert opt.state[m.weight]["step"].item() == 3.0


def test_cpu_sequence_lookup_and_step_match_oracle():
    rng = np.random.default_rng(92)
    (m,) = _modules([("hist", 400, 8)])
    opt = ShardedRowWiseAdagrad([m.weight], lr=0.05, eps=1e-8)
    W0 = m.weight.detach().numpy().copy()
    B, L = 12, 30
    lengths = rng.integers(0, L + 5, size=B)
    ids = np.zeros((B, L), dtype=np.int64)
    for b in range(B):
        k = min(int(lengths[b]), L)
        ids[b, :k] = rng.zipf(1.1, size=k) % 400
    out, mask = sequence_embedding_lookup(m, torch.from_numpy(ids), torch.from_numpy(lengths), target_length=20,
                                          sequence_order="newest_to_oldest")
    ref, rmask = O.sequence_gather(W0, ids, lengths, 20, "newest_to_oldest")
    assert np.array_equal(mask.numpy(), rmask) and np.array_equal(out.detach().numpy(), ref.astype(np.float32))
    g = rng.standard_normal(tuple(out.shape)).astype(np.float32)
    out.backward(torch.from_numpy(g))
    opt.step()
    r, v = O.sequence_grads(ids, lengths, g, 20, "newest_to_oldest")
    r, v = O.coalesce(r, v)
    wexp, aexp = O.rowwise_adagrad(W0, np.zeros(400, np.float32), r, v, 0.05, 1e-8)
    np.testing.assert_allclose(m.weight.detach().numpy(), wexp, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(opt.state[m.weight]["sum"].numpy(), aexp, rtol=1e-5, atol=1e-7)


def _coo(rows, values, size, dtype=torch.float32):
    return torch.sparse_coo_tensor(torch.tensor([rows], dtype=torch.int64), torch.tensor(values, dtype=dtype),
                                   size=size)


def test_cpu_adagrad_lr_decay_and_step_counts():
    """The step count of every parameter with a gradient goes up by one per
    step, and lr_decay scales the rate by 1 / (1 + (step - 1) * lr_decay)
    (src/optim.py:335-341); a parameter without a gradient keeps its count."""

    rng = np.random.default_rng(5)
    w0 = rng.standard_normal((12, 4)).astype(np.float32)
    p = nn.Parameter(torch.from_numpy(w0.copy()))
    idle = nn.Parameter(torch.zeros(3, 4))
    lr, decay, eps = 0.2, 0.5, 1e-8
    opt = ShardedRowWiseAdagrad([p, idle], lr=lr, lr_decay=decay, initial_accumulator_value=0.1, eps=eps)
    W, A = w0.astype(np.float64), np.full(12, 0.1, np.float32)
    for step in range(1, 4):
        rows = rng.integers(0, 12, size=6)
        vals = rng.standard_normal((6, 4)).astype(np.float32)
        p.grad = torch.sparse_coo_tensor(torch.from_numpy(rows).unsqueeze(0), torch.from_numpy(vals), size=p.shape)
        idle.grad = None
        opt.step()
        r, v = O.coalesce(rows, vals.astype(np.float64))
        W, A = O.rowwise_adagrad(W, A, r, v, lr / (1.0 + (step - 1) * decay), eps)
        assert float(opt.state[p]["step"].item()) == float(step)
        assert float(opt.state[idle]["step"].item()) == 0.0
        assert np.allclose(p.detach().numpy(), W, rtol=1e-5, atol=1e-6)
        assert np.allclose(opt.state[p]["sum"].numpy(), A, rtol=1e-5, atol=1e-7)


def test_cpu_adagrad_golden_vectors():
    """The reference tests' cases on CPU parameters (tests/test_rowwise_adagrad.py:40-128)."""

    g = GOLD["rowwise_adagrad_mean_not_sum"]
    p = nn.Parameter(torch.zeros(*g["shape"]))
    opt = ShardedRowWiseAdagrad([p], lr=g["lr"], initial_accumulator_value=0.0, eps=g["eps"])
    p.grad = _coo(g["rows"], g["values"], p.shape).coalesce()
    opt.step()
    for r, a in g["expected_acc"].items():
        assert abs(float(opt.state[p]["sum"][int(r)]) - a) < 1e-6
    for r, w in g["expected_neg_weight"].items():
        assert torch.allclose(p[int(r)].neg(), torch.tensor(w), atol=g["atol"])
    g = GOLD["rowwise_adagrad_duplicates_coalesce"]
    p = nn.Parameter(torch.zeros(*g["shape"]))
    opt = ShardedRowWiseAdagrad([p], lr=g["lr"], initial_accumulator_value=0.0, eps=g["eps"])
    p.grad = _coo(g["rows"], g["values"], p.shape)
    opt.step()
    assert abs(float(opt.state[p]["sum"][3]) - g["expected_acc"]["3"]) < 1e-6
    assert int((opt.state[p]["sum"] != 0).sum()) == g["expected_nonzero_acc_rows"]
    g = GOLD["rowwise_adagrad_empty_noop"]
    p = nn.Parameter(torch.ones(*g["shape"]))
    opt = ShardedRowWiseAdagrad([p], lr=g["lr"], initial_accumulator_value=g["acc0"])
    p.grad = torch.sparse_coo_tensor(torch.empty((1, 0), dtype=torch.int64), torch.empty((0, 2)), size=p.shape)
    opt.step()
    assert torch.equal(p, torch.ones(*g["shape"]))
    assert float(opt.state[p]["step"].item()) == g["expected_step"]
    g = GOLD["rowwise_adagrad_bf16_untouched"]
    p = nn.Parameter(torch.tensor(g["weight"], dtype=torch.bfloat16))
    before = p.detach().clone()
    opt = ShardedRowWiseAdagrad([p], lr=g["lr"], initial_accumulator_value=0.0, eps=g["eps"])
    p.grad = _coo(g["rows"], g["values"], p.shape, dtype=torch.bfloat16).coalesce()
    opt.step()
    for r in g["untouched_rows"]:
        assert torch.equal(p[r], before[r])
    assert abs(float(opt.state[p]["sum"][1]) - g["expected_acc_row1"]) < 1e-6


def test_cpu_errors_follow_the_reference():
    (m,) = _modules([("t", 10, 4)])
    with pytest.raises(IndexError, match=r"embedding 't' received IDs outside \[0, 10\): \[10, -1\]"):
        m(torch.tensor([1, 10, -1]))
    with pytest.raises(TypeError, match="torch.long"):
        m(torch.tensor([1, 2], dtype=torch.int32))
    opt = ShardedRowWiseAdagrad([m.weight], lr=0.1)
    m.weight.grad = torch.zeros_like(m.weight)
    with pytest.raises(RuntimeError, match="row-sparse COO"):
        opt.step()


def test_coalesced_gradient_is_exact_and_marked_coalesced():
    """The default sparse-gradient mode: the lookup's gradient arrives
    coalesced (rows ascending and unique, is_coalesced() true), so the
    trainer's grad.coalesce() (src/train.py:5738, src/optim.py:323-324)
    returns the same tensor; its values are the per-row sums."""

    assert mdl_amd.library.sparse_grad_mode() == "coalesced"
    (m,) = _modules([("t", 50, 4)])
    ids = torch.tensor([7, 3, 7, 0, 9, 3])
    out = m(ids)
    g = torch.randn(out.shape)
    out.backward(g)
    grad = m.weight.grad
    assert grad.is_coalesced()
    assert grad._indices()[0].tolist() == [3, 7, 9]
    assert grad.coalesce() is grad
    dense = torch.zeros(50, 4)
    dense.index_add_(0, ids, g)
    dense[0] = 0  # padding_idx gets no gradient
    torch.testing.assert_close(grad.to_dense(), dense)
    torch.testing.assert_close(grad._values(), dense[[3, 7, 9]])


def test_capacity_gradient_is_a_valid_coo_of_the_coalesced_sum(capacity_grads):
    """The lookup's gradient has one entry per id (a bound known without a
    device read); coalescing it gives the exact coalesced gradient."""

    (m,) = _modules([("t", 50, 4)])
    ids = torch.tensor([7, 3, 7, 0, 9, 3])
    out = m(ids)
    g = torch.randn(out.shape)
    out.backward(g)
    grad = m.weight.grad
    assert grad._indices().size(1) == ids.numel()
    dense = torch.zeros(50, 4)
    dense.index_add_(0, ids, g)
    dense[0] = 0  # padding_idx gets no gradient
    torch.testing.assert_close(grad.to_dense(), dense)
    c = grad.coalesce()
    assert c.indices()[0].tolist() == [3, 7, 9]


def _dense_grad(rows, dim, x, ln, g, mode):
    r, v = O.per_id_grads(x, ln, g.double().numpy(), mode, "exclude")
    dense = np.zeros((rows, dim))
    np.add.at(dense, r, v)
    return torch.from_numpy(dense).float()


@pytest.mark.parametrize("device", ["cpu", pytest.param("cuda", marks=pytest.mark.gpu)])
@pytest.mark.parametrize("grad_mode", ["coalesced", "capacity"])
def test_gradients_reach_parameters_as_autograd_delivers_them(grad_mode, device):
    """The backward stores a first gradient on its parameter itself only
    where autograd's AccumulateGrad would store the same tensor unobserved;
    hooks, autograd.grad, backward(inputs=...), a second backward and a
    table used by two lookups all see what autograd gives them."""

    mode = mdl_amd.library.sparse_grad_mode()
    mdl_amd.library.set_sparse_grad_mode(grad_mode)
    try:
        rng = np.random.default_rng(5)
        a, b, c = (m.to(device) for m in _modules([("a", 40, 4), ("b", 30, 8), ("c", 25, 4)]))
        B = 6
        la = rng.integers(0, 5, size=B)
        xa = rng.integers(0, 40, size=int(la.sum()))
        xb = rng.integers(0, 30, size=B)
        xc1 = rng.integers(0, 25, size=B)
        xc2 = rng.integers(0, 25, size=B)
        ga, gb, gc1, gc2 = (torch.randn(B, d) for d in (4, 8, 4, 4))

        def t(x):
            return torch.from_numpy(x).to(device)

        want = {
            "a": _dense_grad(40, 4, xa, la, ga, "sum"),
            "b": _dense_grad(30, 8, xb, None, gb, "none"),
            "c": _dense_grad(25, 4, xc1, la * 0 + 1, gc1, "sum") + _dense_grad(25, 4, xc2, None, gc2, "none"),
        }

        def run():
            pooled = pooled_embedding_lookup([(a, t(xa), t(la), "sum", "exclude"),
                                              (c, t(xc1), t(np.ones(B, np.int64)), "sum", "exclude")])
            single = grouped_sharded_embedding_lookup([(b, t(xb)), (c, t(xc2))])
            return ((pooled[0].cpu() * ga).sum() + (pooled[1].cpu() * gc1).sum() + (single[0].cpu() * gb).sum()
                    + (single[1].cpu() * gc2).sum())

        mods = {"a": a, "b": b, "c": c}

        def check(name, grad, scale=1.0):
            assert grad is not None and grad.is_sparse and grad.device.type == device
            torch.testing.assert_close(grad.to_dense().cpu(), want[name] * scale)
            if grad_mode == "coalesced" and name != "c" and scale == 1.0:
                assert grad.is_coalesced() and grad.coalesce() is grad

        # plain backward: every table gets its gradient (c: summed over its two
        # lookups), the first ones stored without AccumulateGrad's re-wrap
        with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CPU]) as prof:
            run().backward()
        names = [e.name for e in prof.events()]
        assert names.count("aten::_sparse_coo_tensor_unsafe") == 0
        for k, m in mods.items():
            check(k, m.weight.grad)
        # a second backward accumulates into the existing gradients
        run().backward()
        for k, m in mods.items():
            check(k, m.weight.grad.coalesce(), 2.0)
        # torch.autograd.grad returns the gradients and leaves .grad alone
        for m in mods.values():
            m.weight.grad = None
        got = torch.autograd.grad(run(), [m.weight for m in mods.values()])
        for (k, m), g in zip(mods.items(), got):
            check(k, g.coalesce())
            assert m.weight.grad is None
        # backward(inputs=...) fills only the named parameter
        run().backward(inputs=[b.weight])
        check("b", b.weight.grad)
        assert a.weight.grad is None and c.weight.grad is None
        b.weight.grad = None
        # a tensor hook sees the gradient, a post-accumulate hook runs after it lands
        seen, landed = [], []
        h1 = a.weight.register_hook(lambda g: seen.append(g))
        h2 = b.weight.register_post_accumulate_grad_hook(lambda p: landed.append(p.grad))
        run().backward()
        assert len(seen) == 1 and len(landed) == 1
        check("a", seen[0].coalesce())
        check("a", a.weight.grad)
        check("b", landed[0].coalesce())
        assert landed[0] is b.weight.grad
        h1.remove()
        h2.remove()
    finally:
        mdl_amd.library.set_sparse_grad_mode(mode)


@pytest.mark.parametrize("device", ["cpu", pytest.param("cuda", marks=pytest.mark.gpu)])
def test_frozen_table_in_a_grouped_lookup_gets_no_gradient(device):
    """A table with requires_grad=False looked up beside trainable ones gets
    no gradient; the trainable ones get theirs."""

    a, b = (m.to(device) for m in _modules([("a", 20, 4), ("b", 20, 4)]))
    b.weight.requires_grad_(False)
    outs = grouped_sharded_embedding_lookup([(a, torch.tensor([1, 2, 2], device=device)),
                                             (b, torch.tensor([3, 3], device=device))])
    torch.autograd.backward(outs, [torch.ones_like(o) for o in outs])
    assert b.weight.grad is None
    dense = a.weight.grad.coalesce().to_dense().cpu()
    assert dense[1].tolist() == [1.0] * 4 and dense[2].tolist() == [2.0] * 4 and float(dense.abs().sum()) == 12.0


def test_modules_compile_with_their_gradients(capacity_grads):
    """torch.compile (full graph, AOT autograd) traces the modules' lookups:
    fake tensors take the op's registered autograd, and the compiled step's
    gradients equal the eager ones."""

    a, b = _modules([("a", 30, 4), ("b", 20, 8)])
    for m in (a, b):
        m.validate_indices = False  # the host-side check reads a device count

    def fn(x, y, ln):
        o = pooled_embedding_lookup([(a, x, ln, "mean", "exclude")])[0]
        s = grouped_sharded_embedding_lookup([(b, y)])[0]
        return (o * 2).sum() + (s * 3).sum()

    x, ln, y = torch.tensor([1, 2, 3, 4, 5]), torch.tensor([2, 3]), torch.tensor([3, 3, 7])
    fn(x, y, ln).backward()
    want = [m.weight.grad.coalesce().to_dense() for m in (a, b)]
    a.weight.grad = b.weight.grad = None
    torch.compile(fn, backend="aot_eager", fullgraph=True)(x, y, ln).backward()
    for m, w in zip((a, b), want):
        torch.testing.assert_close(m.weight.grad.coalesce().to_dense(), w)


def test_cpu_fused_rowwise_adagrad_update_public_function():
    """``fused_rowwise_adagrad_update`` on CPU tensors (the op's CPU kernel,
    the reference's CPU update rule src/optim.py:359-376) on the golden case of
    tests/test_rowwise_adagrad.py:40-62, with fp32 and bf16 values."""

    from mdl_amd.optim import fused_rowwise_adagrad_update

    g = GOLD["rowwise_adagrad_mean_not_sum"]
    for vdtype in (torch.float32, torch.bfloat16):
        p = torch.zeros(*g["shape"])
        acc = torch.zeros(g["shape"][0])
        fused_rowwise_adagrad_update(p, acc, torch.tensor(g["rows"]), torch.tensor(g["values"], dtype=vdtype),
                                     lr=g["lr"], eps=g["eps"])
        for r, a in g["expected_acc"].items():
            assert abs(float(acc[int(r)]) - a) < 1e-6
        for r, w in g["expected_neg_weight"].items():
            assert torch.allclose(p[int(r)].neg(), torch.tensor(w), atol=g["atol"])
