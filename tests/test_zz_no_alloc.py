"""The allocation-free fused backward (mdl_backward_adagrad_noalloc) against
mdl_backward_adagrad with a caller workspace, through the C ABI.

Both run the same kernels in the same fixed summation order, so the updated
weights and accumulators must agree bit for bit -- on two calls in a row on
the same GPU, the second with a smaller input (the static scratch keeps the
first call's contents).  A call whose workspace exceeds the static scratch
is refused before anything is launched.
"""

import sys

import numpy as np
import pytest
import torch

from mdl_amd import _lib, ops

pytestmark = pytest.mark.gpu


def announce(*parts):
    print("CASE", *parts, flush=True)
    sys.stdout.flush()


def _group(device, seed, B, max_len):
    """Two identical copies of a three-table group and one forward batch."""

    rng = np.random.default_rng(seed)
    rows, dims, pools = [4000, 900, 20000], [32, 16, 64], ["mean", "none", "sum"]
    W = [rng.standard_normal((r, d)).astype(np.float32) for r, d in zip(rows, dims)]
    A = [rng.random(r).astype(np.float32) for r in rows]
    ids, lens = [], []
    for t, p in enumerate(pools):
        if p == "none":
            ids.append(rng.zipf(1.1, size=B) % rows[t])
            lens.append(None)
        else:
            ln = rng.integers(0, max_len + 1, size=B)
            ids.append(rng.zipf(1.1, size=int(ln.sum())) % rows[t])
            lens.append(ln)
    grads = [rng.standard_normal((B, d)).astype(np.float32) for d in dims]
    copies = []
    for _ in range(2):
        tabs = [torch.from_numpy(w.copy()).to(device) for w in W]
        accs = [torch.from_numpy(a.copy()).to(device) for a in A]
        plan = ops.GroupPlan()
        for t, p in enumerate(pools):
            plan.add_feature(tabs[t], pooling=p, null_policy="exclude", state=accs[t])
        res = ops.grouped_forward(
            plan, [torch.from_numpy(x.astype(np.int64)).to(device) for x in ids],
            [None if ln is None else torch.from_numpy(ln).to(device) for ln in lens], with_backward=True,
        )
        copies.append((plan, res, tabs, accs))
    return copies, [torch.from_numpy(g).to(device) for g in grads]


def _backward(plan, res, grads, lr, eps, noalloc):
    lib = _lib.lib()
    device = res.device
    feats, keep = ops._attach_grads(res, grads)
    tables = ops._tables_array(plan, feats)
    fd = ops.upload(feats, device)
    td = ops.upload(tables, device)
    n = res.num_ids
    classes = ops.table_classes(tables)
    stream = torch.cuda.current_stream(device).cuda_stream
    args = (fd.data_ptr(), len(feats), td.data_ptr(), len(tables), plan.max_dim, res.keys.data_ptr(),
            res.payload.data_ptr(), n, None, plan.key_bits, ops._ptr(res.bag_count), lr, eps, None)
    if noalloc:
        rc = lib.mdl_backward_adagrad_noalloc(*args, classes, stream)
    else:
        ws = torch.empty(lib.mdl_backward_workspace_bytes(n, len(tables), plan.max_dim), dtype=torch.uint8,
                         device=device)
        rc = lib.mdl_backward_adagrad(*args, ws.data_ptr(), ws.numel(), classes, stream)
    _lib.check(rc, "backward")
    torch.cuda.synchronize()
    del keep


@pytest.mark.parametrize("seed", [0, 1])
def test_noalloc_backward_matches_workspace_call(device, seed):
    lib = _lib.lib()
    assert lib.mdl_noalloc_scratch_bytes() == 64 << 20
    lr, eps = 0.03, 1e-8
    # the larger call first, then a smaller one on the same static scratch
    for k, (B, max_len) in enumerate([(4096, 24), (700, 6)]):
        announce("noalloc", seed, k, B, max_len)
        copies, grads = _group(device, 10 * seed + k, B, max_len)
        (plan_a, res_a, tabs_a, accs_a), (plan_b, res_b, tabs_b, accs_b) = copies
        assert res_a.num_ids == res_b.num_ids
        before = [t.clone() for t in tabs_a]
        _backward(plan_a, res_a, grads, lr, eps, noalloc=False)
        _backward(plan_b, res_b, grads, lr, eps, noalloc=True)
        for t in range(len(tabs_a)):
            assert torch.equal(tabs_a[t], tabs_b[t]), f"call {k}: table {t}"
            assert torch.equal(accs_a[t], accs_b[t]), f"call {k}: accumulator {t}"
            assert not torch.equal(tabs_a[t], before[t]), f"call {k}: table {t} was not updated"


def test_noalloc_refuses_calls_beyond_its_scratch(device):
    lib = _lib.lib()
    n = 8_000_000
    assert lib.mdl_backward_workspace_bytes(n, 200, 128) > lib.mdl_noalloc_scratch_bytes()
    rc = lib.mdl_backward_adagrad_noalloc(None, 1, None, 200, 128, None, None, n, None, 31, None, 0.1, 1e-8,
                                          None, 0, None)
    assert rc == -4 and b"static scratch" in lib.mdl_last_error()
