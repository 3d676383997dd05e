"""Sparse gradient clipping on the GPU: the ``_clip_sparse_grad_norm``
drop-in (src/train.py:5788-5826) and the clip fused into the backward of
``SparseStep``, checked against the CPU oracle."""

import sys

import numpy as np
import pytest
import torch

from mdl_amd import ops
from mdl_amd.clip import _clip_sparse_grad_norm, _gradient_squared_norm, _gradient_values, _scale_gradients
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def announce(*parts):
    print("CASE", *parts, flush=True)
    sys.stdout.flush()


def _sparse_param(rng, rows, dim, n, dtype, device, coalesced):
    p = torch.nn.Parameter(torch.zeros(rows, dim, dtype=dtype, device=device))
    idx = rng.integers(0, rows, size=n)
    if coalesced:
        idx = np.unique(idx)
    vals = torch.from_numpy(rng.standard_normal((idx.size, dim)).astype(np.float32)).to(device=device, dtype=dtype)
    g = torch.sparse_coo_tensor(torch.from_numpy(idx).view(1, -1).to(device), vals, (rows, dim))
    if coalesced:
        g = g.coalesce()
    p.grad = g
    return p


def _dense_values(p, absolute=False):
    """Coalesced (rows, values) of a sparse grad computed on the CPU, fp64
    (of the absolute values: the scale of the fp32 rounding of each sum)."""

    g = p.grad.detach().cpu().double()
    if absolute:
        g = torch.sparse_coo_tensor(g._indices(), g._values().abs(), g.shape)
    g = g.coalesce()
    return g.indices()[0].numpy(), g.values().numpy()


@pytest.mark.parametrize("max_norm", [0.25, 1e6])
def test_clip_sparse_grad_norm_matches_oracle(device, max_norm):
    announce("clip_dropin", max_norm)
    rng = np.random.default_rng(41)
    replicated = [_sparse_param(rng, 500, 16, 3000, torch.float32, device, coalesced=False),
                  _sparse_param(rng, 64, 32, 40, torch.float32, device, coalesced=True)]
    sharded = [_sparse_param(rng, 1000, 8, 2000, torch.float32, device, coalesced=False)]
    dense = torch.nn.Parameter(torch.zeros(7, 3, device=device))
    dense.grad = torch.randn(7, 3, device=device)
    before = [_dense_values(p) for p in replicated + sharded]
    scales = [_dense_values(p, absolute=True)[1] for p in replicated + sharded]
    dense_before = dense.grad.double().cpu().numpy()
    # coalesced on the device and stored back; the clip below reuses them
    snapshot = [v.clone() for v in _gradient_values(replicated + sharded)]
    norm = _clip_sparse_grad_norm(replicated + [dense], sharded, max_norm)
    want, total, coef = O.clip_grad_norm([v for _, v in before] + [dense_before], max_norm)
    assert norm.shape == () and norm.dtype == torch.float32
    assert abs(float(norm) - total) <= 1e-5 * total
    for p, (rows, _), w, sc in zip(replicated + sharded, before, want, scales):
        assert p.grad.is_coalesced()
        assert np.array_equal(p.grad.indices()[0].cpu().numpy(), rows)
        # fp32 sums in input order: error within a few ulps of sum |terms|
        err = np.abs(p.grad.values().cpu().numpy() - w)
        assert np.all(err <= 1e-5 * np.abs(w) + 1e-6 * sc * coef + 1e-12)
    np.testing.assert_allclose(dense.grad.cpu().numpy(), want[-1], rtol=2e-5, atol=1e-7)
    if max_norm > total:  # coefficient 1: the values are left bit-identical
        for p, v in zip(replicated + sharded, snapshot):
            assert torch.equal(p.grad.values(), v)


def test_scale_is_the_dtype_multiply_of_torch(device):
    """bf16 grads are scaled by the coefficient cast to bf16, one rounding."""

    announce("clip_scale_bits")
    rng = np.random.default_rng(42)
    grads = [torch.from_numpy(rng.standard_normal(n).astype(np.float32)).to(device=device, dtype=dt)
             for n, dt in [(1001, torch.bfloat16), (4096, torch.bfloat16), (333, torch.float32), (65536, torch.float32)]]
    grads.append(torch.randn(64, device=device).to(torch.bfloat16)[1:])  # unaligned start
    coef = torch.tensor([0.3712], device=device)
    expect = [(g.cpu() * coef.cpu().to(g.dtype)) for g in grads]
    _scale_gradients(grads, coef)
    for g, e in zip(grads, expect):
        assert torch.equal(g.cpu(), e)


def test_squared_norm_is_deterministic_and_matches_fp64(device):
    announce("clip_sumsq")
    rng = np.random.default_rng(43)
    grads = [torch.from_numpy(rng.standard_normal(n).astype(np.float32)).to(device) for n in (5, 100003, 1 << 20)]
    grads.append(torch.from_numpy(rng.standard_normal(70001).astype(np.float32)).to(device).to(torch.bfloat16))
    a = _gradient_squared_norm(grads, device)
    b = _gradient_squared_norm(grads, device)
    assert a.shape == () and torch.equal(a, b)
    ref = sum(float((g.double().cpu() ** 2).sum()) for g in grads)
    assert abs(float(a) - ref) <= 1e-5 * ref
    empty = _gradient_squared_norm([], device)
    assert float(empty) == 0.0


def test_gradient_values_coalesces_and_stores_back(device):
    announce("clip_values")
    rng = np.random.default_rng(44)
    p = _sparse_param(rng, 50, 4, 500, torch.float32, device, coalesced=False)
    rows, vals = _dense_values(p)
    (v,) = _gradient_values([p])
    assert p.grad.is_coalesced()
    assert np.array_equal(p.grad.indices()[0].cpu().numpy(), rows)
    np.testing.assert_allclose(v.cpu().numpy(), vals, rtol=1e-5, atol=1e-6)


def _clipped_step_oracle(W, pools, ids, lens, grad, cols, dims, lr, eps, max_norm):
    coalesced = []
    for t, (p, x, ln) in enumerate(zip(pools, ids, lens)):
        g = grad[:, cols[t]: cols[t] + dims[t]]
        r, v = O.per_id_grads(x, ln, g, p, "exclude")
        coalesced.append(O.coalesce(r, v))
    scaled, total, coef = O.clip_grad_norm([v for _, v in coalesced], max_norm)
    out = []
    for t, ((r, _), v) in enumerate(zip(coalesced, scaled)):
        out.append(O.rowwise_adagrad(W[t], np.zeros(W[t].shape[0], np.float32), r, v, lr, eps))
    return out, total


@pytest.mark.parametrize("max_norm", [0.05, 1e6])
def test_fused_clip_step_matches_oracle(device, max_norm):
    """SparseStep.step(clip_norm=...): sort, squared norm of the coalesced
    gradient, clip coefficient and the scaled Adagrad apply, all on device."""

    from mdl_amd.sparse_step import SparseStep

    announce("clip_fused_step", max_norm)
    rng = np.random.default_rng(45)
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
    st.forward()
    st.sort()
    norm, coef = st.clip(max_norm)
    st.apply(0.02, 1e-8, coef)
    want, total = _clipped_step_oracle(W, pools, ids, lens, grad.cpu().numpy().astype(np.float64), cols, dims,
                                       0.02, 1e-8, max_norm)
    assert abs(float(norm) - total) <= 1e-5 * total
    if max_norm > total:
        assert float(coef) == 1.0
    for t in range(len(rows)):
        np.testing.assert_allclose(tabs[t].cpu().numpy(), want[t][0], rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(accs[t].cpu().numpy(), want[t][1], rtol=1e-5, atol=1e-9)
    # the squared norm is a fixed-order sum: the same bits on a second pass
    first = norm.clone()
    st.forward()
    st.sort()
    norm2, _ = st.clip(max_norm)
    assert torch.equal(first, norm2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_live_row_spans_cover_only_their_live_rows(device, dtype):
    """A span with a device row count (mdl_span.live_rows, C ABI 6) sums and
    scales only its first rows, clamped to [0, rows]; its sum of squares has
    the bits of a span of exactly those rows (the slices follow the live
    element count), and rows past the count keep their bits."""

    from mdl_amd import ops

    torch.manual_seed(11)
    rows, dim = 1000, 24
    x = torch.randn(rows, dim, device=device).to(dtype)
    for live in (0, 1, 377, rows, rows + 5, -3):
        count = torch.tensor([live], dtype=torch.int64, device=device)
        k = min(max(live, 0), rows)
        got = ops.grad_sumsq([x], device, live_rows=[count])
        want = ops.grad_sumsq([x[:k].contiguous()], device) if k else torch.zeros(1, device=device)
        assert torch.equal(got, want), (live, float(got), float(want))
        y = x.clone()
        coef = torch.tensor([0.37], dtype=torch.float32, device=device)
        ops.scale_([y], coef, live_rows=[count])
        z = x[:k].clone()
        if k:
            ops.scale_([z], coef)
        assert torch.equal(y[:k], z) and torch.equal(y[k:], x[k:]), live
