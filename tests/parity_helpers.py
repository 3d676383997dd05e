"""Shared checks of the full-size parity tests: compact oracle tables over
the touched rows, first-order tolerances of fp32 summation, and bit-exact
checksums of every untouched row."""

import gc
import sys

import numpy as np
import torch

from oracle import oracle as O

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


class ErrorStats:
    """Observed error against |ref|, per category (e.g. "c1 weights"): the
    worst relative error |got - ref| / |ref| over elements with ref != 0, the
    same over the well-conditioned elements (|ref| at least half the
    magnitude the bound uses, the sum of |terms| where the check has one: a
    condition number of at most 2, where fp32 summation's error stays near
    the unit roundoff times the term count),
    how many elements of each exceed the plain relative tolerance, and the
    worst ratio of the error to the bound the check applies (<= 1 passes).
    The full-size tests print one line per category, so each run records how
    close the results come to the plain 1e-5 / 1e-2 relative figures, beside
    the first-order bounds over |terms| that they are checked against."""

    def __init__(self):
        self.cats: dict[str, dict] = {}

    def add(self, what: str, err, ref, bound, rtol: float, scale=None):
        cat = " ".join(what.split()[:1] + [w for w in what.split()[1:] if not w.isdigit()][-1:])
        c = self.cats.setdefault(cat, {"n": 0, "nonzero": 0, "over_rtol": 0, "worst_rel": 0.0, "kept": 0,
                                       "kept_over_rtol": 0, "kept_worst_rel": 0.0, "worst_bound_ratio": 0.0,
                                       "rtol": rtol})
        mag = np.abs(ref)
        nz = mag > 0
        rel = np.where(nz, err / np.where(nz, mag, 1.0), 0.0)
        kept = nz & (mag >= 0.5 * (mag if scale is None else scale))
        c["n"] += int(err.size)
        c["nonzero"] += int(nz.sum())
        c["over_rtol"] += int((rel > rtol).sum())
        c["kept"] += int(kept.sum())
        c["kept_over_rtol"] += int((kept & (rel > rtol)).sum())
        if err.size:
            c["worst_rel"] = max(c["worst_rel"], float(rel.max()))
            if kept.any():
                c["kept_worst_rel"] = max(c["kept_worst_rel"], float(rel[kept].max()))
            c["worst_bound_ratio"] = max(c["worst_bound_ratio"], float((err / bound).max()))

    def report(self, prefix: str = ""):
        for cat, c in sorted(self.cats.items()):
            if prefix and not cat.startswith(prefix):
                continue
            say("ERR", cat, f"elements {c['n']}", f"worst |err|/|ref| {c['worst_rel']:.3e}",
                f"over {c['rtol']:g} relative: {c['over_rtol']} of {c['nonzero']};",
                f"well-conditioned: worst {c['kept_worst_rel']:.3e}, over {c['rtol']:g}: {c['kept_over_rtol']} of "
                f"{c['kept']};", f"worst err/bound {c['worst_bound_ratio']:.3f}")


STATS = ErrorStats()


def assert_close(got, ref, rtol, atol, scale=None, what=""):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    err = np.abs(got - ref)
    mag = np.abs(ref) if scale is None else np.maximum(np.abs(ref), np.asarray(scale, dtype=np.float64))
    bound = atol + rtol * mag
    STATS.add(what, err, ref, bound, rtol, None if scale is None else mag)
    bad = err > bound
    assert not bad.any(), f"{what}: {int(bad.sum())} mismatches, worst excess {float((err - bound).max())}"


def _check_update(what, w_post, a_post, w_pre, a_pre, rows, g, s, lr, eps, rtol, atol_w, is_bf16, acc_rtol=1e-5):
    """Touched rows against the oracle's update of the coalesced gradient.

    ``g`` is the oracle's coalesced gradient (fp64) of local ``rows`` and
    ``s`` the same coalesce over |terms|.  fp32 summation puts at most about
    rtol * s on each gradient element, so the accumulator
    a = a0 + sum(g^2)/dim is compared relative to a0 + sum(s^2)/dim, and the
    weight w = w0 - lr * g / (sqrt(a) + eps) relative to |w| plus the
    first-order effect of both errors:
    lr * (s + |g| * a_scale / (2 sqrt(a) (sqrt(a) + eps))) / (sqrt(a) + eps).
    Rows without a gradient must not change at all.  ``acc_rtol`` is the
    accumulators' relative tolerance: 1e-5 where the gradient is summed in
    fp32 all the way to the update; a gradient stored in a bf16 table's dtype
    on the way (the drop-in's sparse gradients) takes the bf16 tolerance.
    """

    w_ref, a_ref = O.rowwise_adagrad(w_pre, a_pre, rows, g, lr, eps, is_bf16=is_bf16)
    dim = w_pre.shape[1]
    untouched = np.ones(w_pre.shape[0], dtype=bool)
    untouched[rows] = False
    assert np.array_equal(w_post[untouched], w_pre[untouched]), f"{what}: rows without gradient changed"
    assert np.array_equal(a_post[untouched], a_pre[untouched]), f"{what}: state without gradient changed"
    a_scale = a_pre[rows].astype(np.float64) + (s * s).sum(1) / dim
    assert_close(a_post[rows], a_ref[rows], acc_rtol, 1e-7, a_scale, what + " accumulators")
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
