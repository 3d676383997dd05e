"""Benchmark of the MI355X sparse path: fused forward + backward + row-wise
Adagrad over one synthetic batch per step.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c1]

Prints one JSON line.  ``value`` is looked-up (non-padding) rows per second
of the headline config's whole step (c1 by default), timed between device
synchronisations with every input already resident in HBM; each step binds a
different batch (its own ids and bag lengths) to the one step object.
``roofline`` reports the dominant kernel's algorithmic bytes per launch over
its HIP-event-measured duration against MI355X's 8 TB/s; ``cpu_baseline``
times the reference path's PyTorch CPU restatement (oracle/torch_path.py) on
this run's first batch with every CPU thread the process may use.
``configs`` then holds the same measurements for every other BASELINE
config, run one after another with their tables freed in between (c0 with
its own full-size CPU baseline).

Workloads:
  c1  RankMixer-scale step (default): 200 features (150 single-valued, 50 bags
      of 1..32 ids), batch 8192, table rows log-uniform in [1e3, 5e7] scaled to
      1.5e9 rows in total, dims {16,32,64,128} (tables above 1e7 rows use 16/32
      so fp32 tables + state fit one GPU), fp32, Zipf(1.1) ids, mean pooling.
  c3  c1 with bf16 tables (fp32 accumulation and state).
  c0  32 tables x 1e6 x 64 fp32, batch 4096, Poisson(3) bags clipped to
      [1,16], Zipf(1.05) raw ids over 2^40 bucketed mod table size, sum pooling.
  c2  4 sequences of 64..2000 ids padded to 2048, 2e8 x 64 fp32 tables,
      batch 1024, Zipf(0.9) with 10% repeats, right-aligned windows + mask.
  c4  capacity: 8 x 1.875e8 x 64 bf16 tables (1.5e9 rows) with uniform ids
      plus 24 x 1e5 x 32 with Zipf(1.2), batch 16384, sum pooling.
"""

from __future__ import annotations

import argparse
import gc
import json
import os
import platform
import sys
import time
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "looked-up rows/s + achieved HBM GB/s (fwd+bwd+Adagrad) at batch 8192, 1 GPU"
PEAK_HBM_GBPS = 8000.0


# ------------------------------------------------------------- workloads --


@dataclass
class Feature:
    table: int
    pooling: str  # "none" | "sum" | "mean"
    bag_len: tuple[int, int] | None  # uniform [lo, hi] bag length; None = single-valued
    poisson: float | None = None


@dataclass
class Workload:
    name: str
    batch: int
    rows: list[int]
    dims: list[int]
    dtype: str  # "fp32" | "bf16"
    features: list[Feature]
    zipf: list[float]  # per table; 0 = uniform
    raw_bits: int | None = None  # raw ids drawn over 2^raw_bits then bucketed mod rows
    kind: str = "pooled"  # "pooled" | "sequence"
    seq_len: tuple[int, int, int] | None = None  # (min len, max len, padded length) for sequences
    repeat_frac: float = 0.0  # share of sequence positions that repeat an earlier id of the row
    lr: float = 0.01
    eps: float = 1e-8
    notes: dict = field(default_factory=dict)


def workload_c1(dtype: str = "fp32") -> Workload:
    rng = np.random.default_rng(2024)
    n_tables = 200
    log_rows = rng.uniform(np.log(1e3), np.log(5e7), size=n_tables)
    rows = np.exp(log_rows)
    rows = np.maximum((rows * (1.5e9 / rows.sum())).astype(np.int64), 1000)
    dims = rng.choice([16, 32, 64, 128], size=n_tables)
    big = rows > 10_000_000
    dims[big] = rng.choice([16, 32], size=int(big.sum()))
    esize = 4 if dtype == "fp32" else 2
    # keep weights + fp32 state under 250 GB: narrow the largest tables first
    order = np.argsort(-rows)
    k = 0
    while int((rows * dims * esize + rows * 4).sum()) > 250e9 and k < n_tables:
        dims[order[k]] = 16
        k += 1
    feats = []
    perm = rng.permutation(n_tables)
    bag_tables = set(perm[:50].tolist())
    for t in range(n_tables):
        if t in bag_tables:
            feats.append(Feature(table=t, pooling="mean", bag_len=(1, 32)))
        else:
            feats.append(Feature(table=t, pooling="none", bag_len=None))
    return Workload(
        name="c1" if dtype == "fp32" else "c3",
        batch=8192,
        rows=rows.tolist(),
        dims=dims.tolist(),
        dtype=dtype,
        features=feats,
        zipf=[1.1] * n_tables,
        notes={"table_rows_total": int(rows.sum())},
    )


def workload_c0() -> Workload:
    feats = [Feature(table=t, pooling="sum", bag_len=(1, 16), poisson=3.0) for t in range(32)]
    return Workload(
        name="c0", batch=4096, rows=[1_000_000] * 32, dims=[64] * 32, dtype="fp32", features=feats,
        zipf=[1.05] * 32, raw_bits=40,
    )


def workload_c2() -> Workload:
    feats = [Feature(table=t, pooling="none", bag_len=None) for t in range(4)]
    return Workload(
        name="c2", batch=1024, rows=[200_000_000] * 4, dims=[64] * 4, dtype="fp32", features=feats,
        zipf=[0.9] * 4, kind="sequence", seq_len=(64, 2000, 2048), repeat_frac=0.1,
    )


def workload_c4() -> Workload:
    # 1.5e9 rows in total over the 8 large bf16 tables (192 GB), plus 24 small
    feats = [Feature(table=t, pooling="sum", bag_len=(1, 1)) for t in range(32)]
    rows = [187_500_000] * 8 + [100_000] * 24
    dims = [64] * 8 + [32] * 24
    return Workload(
        name="c4", batch=16384, rows=rows, dims=dims, dtype="bf16", features=feats,
        zipf=[0.0] * 8 + [1.2] * 24,
    )


WORKLOADS = {
    "c1": workload_c1,
    "c3": lambda: workload_c1("bf16"),
    "c0": workload_c0,
    "c2": workload_c2,
    "c4": workload_c4,
}


def bounded_zipf(rng: np.random.Generator, alpha: float, n: int, hi: int) -> np.ndarray:
    """Zipf(alpha) on [1, hi] by inverse CDF over a log-spaced grid (alpha > 0)."""

    if alpha > 1.0 and hi > 1 << 40:
        return rng.zipf(alpha, size=n)
    grid = np.unique(np.logspace(0, np.log10(hi), 4096).astype(np.int64))
    grid = grid[grid >= 1]
    # P(X <= k) ~ H(k, alpha) / H(hi, alpha), H via the integral approximation
    def H(k):
        k = k.astype(np.float64)
        if abs(alpha - 1.0) < 1e-9:
            return np.log(k) + 0.5772156649 + 1 / (2 * k)
        return (k ** (1 - alpha) - 1) / (1 - alpha) + 0.5 * (1 + k ** (-alpha))
    cdf = H(grid) / H(np.array([hi]))[0]
    u = rng.random(n)
    idx = np.searchsorted(cdf, u)
    idx = np.minimum(idx, grid.size - 1)
    lo = np.where(idx > 0, grid[np.maximum(idx - 1, 0)] + 1, 1)
    hi_ = grid[idx]
    return lo + (rng.random(n) * (hi_ - lo + 1)).astype(np.int64)


def draw_ids(rng: np.random.Generator, wl: Workload, t: int, n: int) -> np.ndarray:
    rows = wl.rows[t]
    a = wl.zipf[t]
    if a <= 0:
        return rng.integers(1, rows, size=n)
    if wl.raw_bits:
        raw = bounded_zipf(rng, a, n, 1 << wl.raw_bits)
    elif a <= 1.0:
        raw = bounded_zipf(rng, a, n, rows - 1)
    else:
        raw = rng.zipf(a, size=n)
    # the reference benchmark's id rule: 1 + (z - 1) mod (N - 1), src/benchmark.py:1246-1250
    return 1 + (raw - 1) % (rows - 1)


def draw_batch(rng: np.random.Generator, wl: Workload):
    """Per-feature ids and bag lengths (None for single-valued features).

    Sequence workloads return right-padded ``[B, L]`` ids and ``[B]`` lengths."""

    if wl.kind == "sequence":
        lo, hi, pad = wl.seq_len
        ids, lengths = [], []
        for f in wl.features:
            ln = rng.integers(lo, hi + 1, size=wl.batch)
            flat = draw_ids(rng, wl, f.table, int(ln.sum()))
            mat = np.zeros((wl.batch, pad), dtype=np.int64)
            pos = 0
            for b in range(wl.batch):
                row = flat[pos: pos + ln[b]].copy()
                pos += ln[b]
                k = int(wl.repeat_frac * ln[b])
                if k and ln[b] > 1:
                    dst = rng.integers(1, ln[b], size=k)
                    src = (rng.random(k) * dst).astype(np.int64)  # an earlier position of the row
                    row[dst] = row[src]
                mat[b, : ln[b]] = row
            ids.append(mat)
            lengths.append(ln)
        return ids, lengths
    ids, lengths = [], []
    for f in wl.features:
        if f.bag_len is None:
            ln = None
            n = wl.batch
        else:
            lo, hi = f.bag_len
            if f.poisson:
                ln = np.clip(rng.poisson(f.poisson, size=wl.batch), lo, hi)
            else:
                ln = rng.integers(lo, hi + 1, size=wl.batch)
            n = int(ln.sum())
        ids.append(draw_ids(rng, wl, f.table, n))
        lengths.append(ln)
    return ids, lengths


def algorithmic_bytes(wl: Workload, ids, lengths) -> dict:
    """Per-step algorithmic HBM bytes and their parts.  Pooled workloads:
    sum over tables t of 16 n_t + 16 (b_t + 1) + 3 U_t D_t s_w + 8 U_t, plus
    2 B D_f 4 per feature f -- ids and offsets read by the forward and the
    backward, each distinct row read by the lookup and read and written by
    the update, its fp32 state read and written, the pooled output written
    and its gradient read (n_t ids, b_t bags and U_t distinct rows of table
    t, s_w bytes per weight).  The output and its gradient are counted at
    their element size s_o, which is the tables' (4 fp32, 2 bf16): the
    step's buffers hold bf16 for bf16 tables, so 2 B D_f s_o per feature.
    Sequences replace the pooled output by the padded window and its mask
    and read the gradient at the valid positions only."""

    esize = 4 if wl.dtype == "fp32" else 2
    if wl.kind == "sequence":
        total = 0
        n_ids = 0
        uniq = 0
        fwd_rows = 0
        _, _, pad = wl.seq_len
        for f, mat, ln in zip(wl.features, ids, lengths):
            valid = np.arange(mat.shape[1])[None, :] < ln[:, None]
            x = mat[valid]
            x = x[x != 0]
            u = np.unique(x).size
            n = x.size
            d = wl.dims[f.table]
            n_ids += n
            uniq += u
            fwd_rows += u * d * esize
            # ids + lengths read twice, distinct rows 3x, state, padded output +
            # mask, gradient rows at the valid positions
            total += 16 * n + 16 * (wl.batch + 1) + 3 * u * d * esize + 8 * u
            total += wl.batch * pad * d * esize + wl.batch * pad + n * d * esize
        return {"B_alg": total, "n_ids": n_ids, "unique_rows": uniq, "fwd_unique_row_bytes": fwd_rows,
                "sum_dim": sum(wl.dims[f.table] for f in wl.features)}
    n_t = {}
    uniq_t = {}
    bags_t = {}
    for f, x, ln in zip(wl.features, ids, lengths):
        n_t.setdefault(f.table, []).append(x)
        bags_t[f.table] = bags_t.get(f.table, 0) + (len(ln) if ln is not None else wl.batch)
    total = 0
    fwd_unique_rows_bytes = 0
    n_ids = 0
    for t, xs in n_t.items():
        x = np.concatenate(xs)
        x = x[x != 0]
        u = np.unique(x).size
        uniq_t[t] = u
        n = x.size
        n_ids += n
        d = wl.dims[t]
        total += 16 * n + 16 * (bags_t[t] + 1) + 3 * u * d * esize + 8 * u
        fwd_unique_rows_bytes += u * d * esize
    sum_d = sum(wl.dims[f.table] for f in wl.features)
    # output and gradient in the output dtype (DeviceStep allocates both in
    # the tables' dtype)
    total += 2 * wl.batch * sum_d * esize
    return {
        "B_alg": total,
        "n_ids": n_ids,
        "unique_rows": int(sum(uniq_t.values())),
        "fwd_unique_row_bytes": fwd_unique_rows_bytes,
        "sum_dim": sum_d,
    }


# ---------------------------------------------------------------- device --


class DeviceStep:
    """Tables, persistent buffers, every synthetic batch resident in HBM and
    one SparseStep for all of them: each step binds its batch (packed ids and
    bag lengths) and the step places the features on the device."""

    def __init__(self, wl: Workload, batches, device, layout: str = "slot"):
        import torch

        from mdl_amd import ops
        from mdl_amd.sparse_step import SparseStep

        self.torch = torch
        self.wl = wl
        self.device = device
        wdtype = torch.float32 if wl.dtype == "fp32" else torch.bfloat16
        self.tables = []
        self.states = []
        gen = torch.Generator(device=device)
        gen.manual_seed(1234)
        for r, d in zip(wl.rows, wl.dims):
            w = torch.empty((r, d), dtype=wdtype, device=device)
            w.normal_(0.0, 0.02, generator=gen)
            w[0].zero_()
            self.tables.append(w)
            self.states.append(torch.zeros(r, dtype=torch.float32, device=device))
        self.plan = ops.GroupPlan()
        for f in wl.features:
            self.plan.add_feature(
                self.tables[f.table], pooling=f.pooling, null_policy="exclude", state=self.states[f.table]
            )
        sum_d = sum(wl.dims[f.table] for f in wl.features)
        out_views, grad_views = [], []
        if layout == "slot":
            # pooled outputs go straight into the token-slot buffer [B, sum(dim)]
            self.out = torch.empty((wl.batch, sum_d), dtype=wdtype, device=device)
            self.grad = torch.empty((wl.batch, sum_d), dtype=wdtype, device=device)
            self.grad.normal_(0.0, 1.0, generator=gen)
            col = 0
            for f in wl.features:
                d = wl.dims[f.table]
                out_views.append(self.out[:, col: col + d])
                grad_views.append(self.grad[:, col: col + d])
                col += d
        else:
            # one [B, dim] output per feature, as the grouped lookup returns them
            # (src/embeddings.py:1646-1751, pooled per feature src/model.py:590-678)
            self.out = torch.empty(wl.batch * sum_d, dtype=wdtype, device=device)
            self.grad = torch.empty(wl.batch * sum_d, dtype=wdtype, device=device)
            self.grad.normal_(0.0, 1.0, generator=gen)
            off = 0
            for f in wl.features:
                d = wl.dims[f.table]
                out_views.append(self.out[off: off + wl.batch * d].view(wl.batch, d))
                grad_views.append(self.grad[off: off + wl.batch * d].view(wl.batch, d))
                off += wl.batch * d
        self.err = torch.zeros(1, dtype=torch.int32, device=device)
        # device-resident batches: packed ids + concatenated lengths (an unpooled
        # feature contributes one pseudo-bag holding all its ids)
        self.batches = []
        self.batch_counts = []
        for ids, lengths in batches:
            self.batch_counts.append([(int(x.size), 0 if ln is None else int(ln.size)) for x, ln in zip(ids, lengths)])
            parts = [ln if ln is not None else np.array([x.size]) for x, ln in zip(ids, lengths)]
            packed = torch.from_numpy(np.concatenate(ids).astype(np.int64)).to(device)
            lens = torch.from_numpy(np.concatenate(parts).astype(np.int64)).to(device)
            self.batches.append((packed, lens))
        ids0, lengths0 = batches[0]
        capacity = max(int(b[0].numel()) for b in self.batches)
        self.st = SparseStep(self.plan, self.batches[0][0], self.batches[0][1], [int(x.size) for x in ids0],
                             [0 if ln is None else int(ln.size) for ln in lengths0], out_views, grad_views,
                             error_count=self.err, capacity=capacity)
        self.steps = [self.st]

    def bind(self, i: int):
        packed, lens = self.batches[i % len(self.batches)]
        self.st.bind(packed, lens)
        return self.st

    def capture(self):
        # A graph reads the buffers it was recorded with: one graph per batch.
        self.graphs = []
        for i in range(len(self.batches)):
            self.bind(i)
            self.st.capture(self.wl.lr, self.wl.eps)
            self.graphs.append(self.st._graph)

    def step(self, i: int, timers=None):
        if timers is None and getattr(self, "graphs", None):
            self.graphs[i % len(self.graphs)].replay()
            return
        st = self.bind(i)
        if timers is None:
            st.step(self.wl.lr, self.wl.eps)
            return
        timers["forward"].start()
        st.forward()
        timers["forward"].stop()
        st.sort()
        timers["apply"].start()
        st.apply(self.wl.lr, self.wl.eps)
        timers["apply"].stop()


class SequenceDeviceStep:
    """Sequence tables, padded windows and one SequenceStep per batch."""

    def __init__(self, wl: Workload, batches, device):
        import torch

        from mdl_amd import ops
        from mdl_amd.sparse_step import SequenceStep

        self.torch = torch
        self.wl = wl
        wdtype = torch.float32 if wl.dtype == "fp32" else torch.bfloat16
        gen = torch.Generator(device=device)
        gen.manual_seed(1234)
        self.tables, self.states = [], []
        for r, d in zip(wl.rows, wl.dims):
            w = torch.empty((r, d), dtype=wdtype, device=device)
            w.normal_(0.0, 0.02, generator=gen)
            w[0].zero_()
            self.tables.append(w)
            self.states.append(torch.zeros(r, dtype=torch.float32, device=device))
        self.plan = ops.GroupPlan()
        for f in wl.features:
            self.plan.add_feature(self.tables[f.table], pooling="none", state=self.states[f.table])
        _, _, pad = wl.seq_len
        self.outs = [torch.empty((wl.batch, pad, wl.dims[f.table]), dtype=wdtype, device=device) for f in wl.features]
        self.masks = [torch.empty((wl.batch, pad), dtype=torch.bool, device=device) for _ in wl.features]
        self.grads = []
        for o in self.outs:
            g = torch.empty_like(o)
            g.normal_(0.0, 1.0, generator=gen)
            self.grads.append(g)
        self.err = torch.zeros(1, dtype=torch.int32, device=device)
        self.batches = []
        for ids, lengths in batches:
            dids = [torch.from_numpy(m).to(device) for m in ids]
            dlen = [torch.from_numpy(ln.astype(np.int64)).to(device) for ln in lengths]
            self.batches.append((dids, dlen))
        self.st = SequenceStep(self.plan, self.batches[0][0], self.batches[0][1], self.outs, self.masks, self.grads,
                               error_count=self.err)
        self.steps = [self.st]

    def bind(self, i: int):
        dids, dlen = self.batches[i % len(self.batches)]
        self.st.bind(dids, dlen)
        return self.st

    def capture(self):
        self.graphs = []
        for i in range(len(self.batches)):
            self.bind(i)
            self.st.capture(self.wl.lr, self.wl.eps)
            self.graphs.append(self.st._graph)

    def step(self, i: int, timers=None):
        if timers is None and getattr(self, "graphs", None):
            self.graphs[i % len(self.graphs)].replay()
            return
        st = self.bind(i)
        if timers is None:
            st.step(self.wl.lr, self.wl.eps)
            return
        timers["forward"].start()
        st.forward()
        timers["forward"].stop()
        st.sort()
        timers["apply"].start()
        st.apply(self.wl.lr, self.wl.eps)
        timers["apply"].stop()


class EventTimer:
    """HIP events recorded on the launch stream around one call's kernels.

    A short spin kernel goes first, so the GPU is still busy while the host
    queues the start event, the call's kernels and the stop event: the pair
    then times the kernels, not the host's launch pace (which shows for
    calls of a few tens of microseconds).  Summarised by the median."""

    SPIN_CYCLES = 2_000_000

    def __init__(self, torch):
        self.torch = torch
        self.pairs = []
        self._open = None

    def start(self):
        stream = self.torch.cuda.current_stream()
        self.torch.cuda._sleep(self.SPIN_CYCLES)
        self._open = self.torch.cuda.Event(enable_timing=True)
        self._open.record(stream)

    def stop(self):
        ev = self.torch.cuda.Event(enable_timing=True)
        ev.record(self.torch.cuda.current_stream())
        self.pairs.append((self._open, ev))

    def median_ms(self):
        self.torch.cuda.synchronize()
        ts = [a.elapsed_time(b) for a, b in self.pairs]
        return float(np.median(ts)) if ts else float("nan")


def aux_measurements(torch, dev, wl, n_ids: float, steps: int, device, batches=None) -> dict:
    """The rows beside the headline step, each timed on its own after it:

    * the clipped step (SparseStep.step with clip_norm: sort, squared norm of
      the coalesced gradient, clip coefficient, apply scaled by it --
      src/train.py:5788-5826), wall clock over ``steps`` steps like the
      headline;
    * the stand-alone row-wise Adagrad update on 1 M unique rows;
    * the drop-in autograd training loop (ShardedEmbedding modules,
      loss.backward(), ShardedRowWiseAdagrad.step()) on the same batches;
    * device bucketing (mdl_bucketize, src/features.py:360-376 and
      src/benchmark.py:1246-1250) of one step's worth of raw int64 ids, HIP
      events around 20 back-to-back launches queued behind a spin kernel, so
      the host's launch time does not show; 16 algorithmic bytes per id
      (read 8, write 8);
    * list features to CSR bags (mdl_bag_truncate), timed the same way.
    """

    from mdl_amd import ops

    out = {}
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        dev.bind(i).step(wl.lr, wl.eps, clip_norm=1.0)
    torch.cuda.synchronize()
    out["clipped_step"] = {
        "ms_per_step": (time.perf_counter() - t0) * 1e3 / steps,
        "clip_norm": 1.0,
        "what": "fused fwd + sort + squared norm + clip coefficient + row-wise Adagrad scaled by it",
    }
    n = int(n_ids)
    gen = torch.Generator(device=device)
    gen.manual_seed(7)
    raw = torch.randint(-(1 << 62), 1 << 62, (n,), dtype=torch.int64, device=device, generator=gen)
    reps = 20
    for mode, buckets in (("pre_hashed", 1 << 20), ("mod", 1_000_003)):
        for _ in range(3):
            ops.bucketize(raw, buckets, mode=mode, validate_nonzero=False)
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(20_000_000)  # holds the stream while the launches queue up
        e0.record()
        for _ in range(reps):
            ops.bucketize(raw, buckets, mode=mode, validate_nonzero=False)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        nbytes = 16.0 * n
        out[f"bucketize_{mode}"] = {
            "n": n, "buckets": buckets, "ms": ms, "alg_bytes": nbytes,
            "achieved_gbps": nbytes / (ms * 1e-3) / 1e9, "frac": nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBPS,
        }
    del raw
    # list features to CSR bags on the device (mdl_bag_truncate: the Arrow
    # truncation, flatten and pre_hashed bucketing of src/dataloader.py:
    # 8565-8665 and :8463-8493): the workload's bag features as raw lists of
    # up to 48 ids per row, the last 32 kept.  Algorithmic bytes: list offsets
    # read, kept raw ids read, capacity-sized ids written (zeros past the
    # kept total), lengths and kept offsets written.
    bag_rows = sum(wl.batch for f in wl.features if f.pooling != "none")
    if bag_rows:
        rng = np.random.default_rng(11)
        lengths = rng.integers(1, 49, size=bag_rows)
        offsets_h = np.zeros(bag_rows + 1, dtype=np.int64)
        np.cumsum(lengths, out=offsets_h[1:])
        n_in = int(offsets_h[-1])
        raw = torch.randint(1, 1 << 62, (n_in,), dtype=torch.int64, device=device, generator=gen)
        offsets = torch.from_numpy(offsets_h).to(device)
        kept = int(np.minimum(lengths, 32).sum())
        call = lambda: ops.bag_truncate(raw, offsets, max_length=32, truncation="tail",  # noqa: E731
                                        bucket="pre_hashed", num_buckets=1 << 20, validate_nonzero=False)
        for _ in range(3):
            call()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(20_000_000)
        e0.record()
        for _ in range(reps):
            call()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        nbytes = 8.0 * (bag_rows + 1) + 8.0 * kept + 8.0 * n_in + 8.0 * bag_rows + 8.0 * (bag_rows + 1)
        out["bag_truncate"] = {
            "rows": bag_rows, "ids_in": n_in, "ids_kept": kept, "ms": ms, "alg_bytes": nbytes,
            "achieved_gbps": nbytes / (ms * 1e-3) / 1e9, "frac": nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBPS,
            "what": "mdl_bag_truncate: tail-truncate to 32, flatten, pre_hashed bucketing (2^20), one call "
                    "(three launches: kept counts, offsets scan, gather)",
        }
        del raw, offsets
    # the stand-alone row-wise Adagrad (fused_rowwise_adagrad_update,
    # src/optim.py:68-108) on 1 M unique rows of the largest table: a weight
    # row read and written, its gradient row read, 8-byte row index and 4-byte
    # accumulator read and written per row
    t = max(range(len(dev.tables)), key=lambda i: dev.tables[i].shape[0])
    w, acc = dev.tables[t], dev.states[t]
    u = min(1 << 20, int(w.shape[0]))
    rows = torch.randperm(int(w.shape[0]), device=device, generator=gen)[:u].sort().values
    vals = torch.randn((u, int(w.shape[1])), device=device, generator=gen)
    for _ in range(3):
        ops.rowwise_adagrad_(w, acc, rows, vals, lr=wl.lr, eps=wl.eps)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(20_000_000)
    e0.record()
    for _ in range(reps):
        ops.rowwise_adagrad_(w, acc, rows, vals, lr=wl.lr, eps=wl.eps)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    esz = w.element_size()
    nbytes = float(u) * (int(w.shape[1]) * (2 * esz + 4) + 16)
    out["rowwise_adagrad"] = {
        "rows": u, "dim": int(w.shape[1]), "table_rows": int(w.shape[0]), "ms": ms, "alg_bytes": nbytes,
        "achieved_gbps": nbytes / (ms * 1e-3) / 1e9, "frac": nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBPS,
    }
    del rows, vals
    # the drop-in autograd path at the same layout: ShardedEmbedding modules
    # over the bench's tables, pooled_embedding_lookup for the bags and
    # grouped_sharded_embedding_lookup for the single-valued features,
    # loss.backward(), ShardedRowWiseAdagrad.step() -- the loop a user of the
    # reference's modules runs (src/model.py:3782-3890, src/train.py:7060-7188),
    # timed under the sync debug mode that raises on any host synchronisation
    if batches is not None:
        k = min(steps, 20)
        out["dropin_step"] = dropin_loop(torch, dev, wl, device, steps=k, mode="capacity")
        out["dropin_step_clipped"] = dropin_loop(torch, dev, wl, device, steps=k, mode="capacity", clip_norm=1.0)
        out["dropin_step_coalesced"] = dropin_loop(torch, dev, wl, device, steps=k, mode="coalesced")
        out["dropin_step_single_thread_autograd"] = dropin_loop(torch, dev, wl, device, steps=k, mode="capacity",
                                                                autograd_threads=False)
    return out


def dropin_loop(torch, dev, wl, device, steps: int = 10, mode: str = "capacity",
                clip_norm: float | None = None, autograd_threads: bool = True) -> dict:
    """The modules' training loop over the bench's tables, in one of the
    sparse-gradient modes: "capacity" (no host read; timed under the sync
    debug mode that raises on any), "coalesced" (exact coalesced gradients,
    one batched read of the row counts per backward).  ``clip_norm`` adds the
    trainer's sparse clip through ``mdl_amd.clip`` between backward and step.
    ``autograd_threads=False`` runs the loop under
    ``torch.autograd.set_multithreading_enabled(False)``: the backward on the
    calling thread instead of autograd's device thread."""

    from torch import nn

    import mdl_amd.library as L
    from mdl_amd.clip import _clip_sparse_grad_norm
    from mdl_amd.embeddings import (EmbeddingShardSpec, ShardedEmbedding, grouped_sharded_embedding_lookup,
                                    pooled_embedding_lookup)
    from mdl_amd.optim import ShardedRowWiseAdagrad

    prev_mode = L.sparse_grad_mode()
    L.set_sparse_grad_mode(mode)

    mods = []
    for t, w in enumerate(dev.tables):
        # built small, then given the resident table (no second copy)
        spec = EmbeddingShardSpec(table_name=f"table_{t}", strategy="row_wise", world_size=1)
        m = ShardedEmbedding(2, int(w.size(1)), table_name=f"table_{t}", shard_spec=spec, collect_stats=False,
                             dtype=w.dtype).to(device)
        m.weight = nn.Parameter(w)
        m.num_embeddings = int(w.size(0))
        mods.append(m)
    opt = ShardedRowWiseAdagrad([m.weight for m in mods], lr=wl.lr, eps=wl.eps)
    for m, acc in zip(mods, dev.states):
        opt.state[m.weight]["sum"] = acc
    cols = np.concatenate([[0], np.cumsum([wl.dims[f.table] for f in wl.features])[:-1]])
    grads = [dev.grad[:, int(c): int(c) + wl.dims[f.table]] for f, c in zip(wl.features, cols)]
    feats = []
    for packed, lens in dev.batches:
        req_pool, req_single, g_pool, g_single = [], [], [], []
        ofs = 0
        lofs = 0
        host_counts = dev.batch_counts[len(feats)]
        for f, feat in enumerate(wl.features):
            n, nb = host_counts[f]
            x = packed[ofs: ofs + n]
            ofs += n
            if feat.pooling == "none":
                req_single.append((mods[feat.table], x))
                g_single.append(grads[f])
                lofs += 1
            else:
                req_pool.append((mods[feat.table], x, lens[lofs: lofs + nb], feat.pooling, "exclude"))
                g_pool.append(grads[f])
                lofs += nb
        feats.append((req_pool, req_single, torch.cat(g_pool + g_single, dim=1)))

    # The model concatenates the per-feature embeddings into its token slots
    # (src/model.py:4395-4420), so one [B, sum(D)] gradient comes back and
    # each feature's share arrives as a column slice of it.
    weights = [m.weight for m in mods]

    def one(i):
        req_pool, req_single, g_tokens = feats[i % len(feats)]
        opt.zero_grad(set_to_none=True)
        outs = pooled_embedding_lookup(req_pool) + grouped_sharded_embedding_lookup(req_single)
        torch.cat(outs, dim=1).backward(g_tokens)
        if clip_norm is not None:
            _clip_sparse_grad_norm([], weights, clip_norm)
        opt.step()

    threads = torch.autograd.set_multithreading_enabled(autograd_threads)
    threads.__enter__()
    try:
        for i in range(2):
            one(i)
        torch.cuda.synchronize()
        clean = mode == "capacity"
        if clean:
            torch.cuda.set_sync_debug_mode("error")
        try:
            t0 = time.perf_counter()
            for i in range(steps):
                one(i)
            torch.cuda.set_sync_debug_mode("default")
            torch.cuda.synchronize()
            ms = (time.perf_counter() - t0) * 1e3 / steps
        except RuntimeError:
            clean = False
            torch.cuda.set_sync_debug_mode("default")
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for i in range(steps):
                one(i)
            torch.cuda.synchronize()
            ms = (time.perf_counter() - t0) * 1e3 / steps
    finally:
        threads.__exit__(None, None, None)
        L.set_sparse_grad_mode(prev_mode)
    grads_what = ("capacity-sized coalesced sparse grads (no host read)" if mode == "capacity" else
                  "exact coalesced sparse grads (is_coalesced, one batched read of the row counts per backward)")
    return {"ms_per_step": ms, "steps": steps, "mode": mode, "clip_norm": clip_norm, "no_host_sync": clean,
            "what": "ShardedEmbedding modules (pooled_embedding_lookup + grouped_sharded_embedding_lookup), "
                    "their outputs concatenated into [B, sum(D)] token slots, backward of one [B, sum(D)] "
                    f"gradient -> {grads_what}, "
                    + ("mdl_amd.clip._clip_sparse_grad_norm, " if clip_norm is not None else "")
                    + "ShardedRowWiseAdagrad.step() (one call, one grouped launch)"
                    + ("; timed steps under torch.cuda.set_sync_debug_mode('error')" if mode == "capacity" else "")
                    + ("" if autograd_threads else
                       "; under torch.autograd.set_multithreading_enabled(False) (backward on the calling thread)")}


# ------------------------------------------------------------ cpu baseline --


# Row caps for hosts whose RAM is smaller than a config's tables.
CPU_ROW_CAP = {"c1": 1 << 20, "c3": 1 << 20, "c2": 1 << 22, "c4": 1 << 22}


def _host_info() -> dict:
    info = {"os_cpu_count": os.cpu_count(), "cpu_model": platform.processor() or platform.machine(), "ram_gb": None}
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                info["cpu_model"] = line.split(":", 1)[1].strip()
                break
        for line in Path("/proc/meminfo").read_text().splitlines():
            if line.startswith("MemTotal"):
                info["ram_gb"] = round(int(line.split()[1]) / 1e6, 1)
                break
    except OSError:
        pass
    return info


def cpu_baseline(wl: Workload, batch, steps: int = 5, warmup: int = 2, row_cap: int | None = None) -> dict:
    """Time the reference path's PyTorch CPU restatement (oracle/torch_path.py:
    F.embedding(sparse=True) -> index_add_ pooling -> autograd -> coalesce()
    -> the CPU row-wise Adagrad branch) on this run's first batch, with every
    CPU thread the process may use; the median of ``steps`` steps after
    ``warmup``.  Tables are full size when the host's RAM exceeds their
    virtual size; otherwise tables above ``row_cap`` rows are capped (the same
    ids bucketed mod the cap, the reference benchmark's rule).  A step reads and writes only the rows its batch touches:
    those get random values (accumulators zero); the rest are never faulted
    in."""

    import torch

    from oracle import torch_path as TP

    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    torch.set_num_threads(threads)
    dtype = torch.float32 if wl.dtype == "fp32" else torch.bfloat16
    esize = 4 if wl.dtype == "fp32" else 2
    cap = row_cap
    if cap is None:
        # Full-size tables whenever the host's RAM exceeds their virtual size
        # (only the touched rows' pages are ever committed); else the cap.
        need = sum(r * (d * esize + 4) for r, d in zip(wl.rows, wl.dims))
        ram = (_host_info()["ram_gb"] or 0) * 1e9
        cap = None if need < 0.8 * ram else CPU_ROW_CAP.get(wl.name, 1 << 20)
    rows = [min(r, cap) if cap else r for r in wl.rows]
    capped = any(r != q for r, q in zip(rows, wl.rows))
    t0 = time.perf_counter()
    # Left unset except the rows the batch touches, which are the only rows a
    # step reads or writes (set below): untouched pages are never faulted in.
    tables = [torch.empty((r, d), dtype=dtype) for r, d in zip(rows, wl.dims)]
    accs = [torch.empty(r, dtype=torch.float32) for r in rows]

    def cap_ids(x, t):
        x = np.asarray(x, dtype=np.int64)
        if rows[t] == wl.rows[t]:
            return torch.from_numpy(x)
        return torch.from_numpy(np.where(x > 0, 1 + (x - 1) % (rows[t] - 1), 0))

    rng = np.random.default_rng(7)
    if wl.kind == "sequence":
        _, _, pad = wl.seq_len
        feats = [TP.Feature(f.table, "none") for f in wl.features]
        ids_t, lens_t, grads = [], [], []
        n_active = 0
        for f, (m, ln) in zip(wl.features, zip(*batch)):
            # the window layout of src/model.py:2989-3020 is a gather of the
            # looked-up rows; time the lookup of every padded position and
            # the gradient of the valid ones (the padding rows get none)
            ids_t.append(cap_ids(m, f.table))
            lens_t.append(None)
            valid = np.arange(m.shape[1])[None, :] < np.asarray(ln)[:, None]
            g = np.zeros(m.shape + (wl.dims[f.table],), dtype=np.float32)
            g[valid] = rng.standard_normal((int(valid.sum()), wl.dims[f.table])).astype(np.float32)
            grads.append(torch.from_numpy(g).to(dtype))
            n_active += int((m[valid] != 0).sum())
    else:
        ids, lengths = batch
        feats = [TP.Feature(f.table, f.pooling) for f in wl.features]
        ids_t = [cap_ids(x, f.table) for f, x in zip(wl.features, ids)]
        lens_t = [None if ln is None else torch.from_numpy(np.asarray(ln, dtype=np.int64)) for ln in lengths]
        grads = [torch.from_numpy(rng.standard_normal((wl.batch, wl.dims[f.table])).astype(np.float32)).to(dtype)
                 for f in wl.features]
        n_active = int(sum(int((np.asarray(x) != 0).sum()) for x in ids))
    gen = torch.Generator().manual_seed(5)
    for f, x in zip(wl.features, ids_t):
        u = torch.unique(x)
        tables[f.table][u] = (torch.randn((u.numel(), wl.dims[f.table]), generator=gen) * 0.02).to(dtype)
        tables[f.table][0].zero_()
        accs[f.table][u] = 0.0
    setup_s = time.perf_counter() - t0
    step = TP.TorchStep(tables, accs, feats)
    times = []
    for i in range(warmup + steps):
        t1 = time.perf_counter()
        step.step(ids_t, lens_t, grads, wl.lr, wl.eps)
        if i >= warmup:
            times.append(time.perf_counter() - t1)
    ms = float(np.median(times)) * 1e3
    info = _host_info()
    total_rows = sum(rows)
    return {
        "value": n_active / (ms * 1e-3),
        "unit": "rows/s",
        "cores": threads,
        "kind": "port",
        "ms_per_step": ms,
        "sample": (f"{wl.name} at full batch {wl.batch} ({n_active} looked-up ids), the bench's first batch; "
                   + (f"tables capped at {cap} rows ({total_rows:.3e} rows in all, ids bucketed mod the cap) "
                      "so they fit host RAM; " if capped else f"full-size tables ({total_rows:.3e} rows); ")
                   + f"PyTorch {torch.__version__} CPU restatement of the reference path (oracle/torch_path.py), "
                   f"median of {steps} steps after {warmup} warmup, torch.set_num_threads({threads}); "
                   f"host: {info['cpu_model']}, os.cpu_count()={info['os_cpu_count']}, "
                   f"{threads} CPUs usable by the process, {info['ram_gb']} GB RAM; table set-up {setup_s:.1f} s"),
        "threads": threads,
        "row_cap": cap if capped else None,
        "host": info,
    }


# ------------------------------------------------------------ rocprof data --
#
# HBM traffic of the dominant kernel comes from two rocprofv3 counter runs of
# this script (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch), each scaled by
# what the same counter reads for a plain 1 GiB device copy measured in the
# same runs (--calibrate-copy):
#   rocprofv3 --pmc FETCH_SIZE -d D1 -o run -- python bench.py --calibrate-copy ...
# (the calibration kernel is torch.neg over 1 GiB: 1 GiB read, 1 GiB written)
#   rocprofv3 --pmc WRITE_SIZE -d D2 -o run -- python bench.py --calibrate-copy ...
#   python bench.py --summarize-pmc D1 D2 --pmc-out profiles/<config>_traffic.json
# The bench line then reports that file's figure as roofline.traffic.

KERNEL_GROUPS = {
    "forward": ("forward_kernel", "sequence_kernel", "sequence_keys_kernel"),
    "apply": ("bwd_reduce_kernel<false", "bwd_reduce_kernel<true"),
    "sort": ("radix_upsweep", "radix_scan", "radix_downsweep"),
}
COPY_BYTES = 1 << 30


def _rocpd_rows(dirs, query):
    import glob
    import sqlite3

    for d in dirs:
        for f in sorted(glob.glob(os.path.join(d, "**", "*.db"), recursive=True)):
            con = sqlite3.connect(f)
            try:
                yield from con.execute(query)
            finally:
                con.close()


def summarize_pmc(dirs, out_path, config, steps_run):
    """FETCH_SIZE / WRITE_SIZE per step of the kernel groups and the copy
    calibration, from rocprofv3 --pmc databases of a bench run that made
    ``steps_run`` step() calls; writes a JSON summary."""

    per = {}
    for name, ctr, val in _rocpd_rows(dirs, "select kernel_name, counter_name, value from counters_collection"):
        per.setdefault(ctr, {}).setdefault(name, []).append(float(val))
    for ctr in ("FETCH_SIZE", "WRITE_SIZE"):
        if ctr not in per:
            raise SystemExit(f"no {ctr} samples under {dirs}")
    copy = [n for n in per["FETCH_SIZE"] if "neg_kernel" in n]
    if not copy:
        raise SystemExit("no copy-kernel calibration samples (run with --calibrate-copy)")
    cname = max(copy, key=lambda n: np.mean(per["FETCH_SIZE"][n]))
    f_kib = float(np.mean(per["FETCH_SIZE"][cname]))
    w_kib = float(np.mean(per["WRITE_SIZE"].get(cname, [float("nan")])))
    scale = {"FETCH_SIZE": COPY_BYTES / (f_kib * 1024), "WRITE_SIZE": COPY_BYTES / (w_kib * 1024)}
    groups = {}
    for g, pats in KERNEL_GROUPS.items():
        tot = {"FETCH_SIZE": 0.0, "WRITE_SIZE": 0.0}
        kernels = {}
        for ctr in tot:
            for n, vals in per[ctr].items():
                if any(p in n for p in pats):
                    k = kernels.setdefault(n.split("(")[0].replace("void ", ""), {})
                    k[ctr + "_KiB"] = float(np.mean(vals))
                    k["dispatches"] = len(vals)
        for k in kernels.values():
            k["dispatches_per_step"] = k["dispatches"] / steps_run
            for ctr in tot:
                tot[ctr] += k.get(ctr + "_KiB", 0.0) * k["dispatches_per_step"]
        # one step's launches of the group: the unit bench.py times per kernel
        # group (all features' forward launches, all sort passes)
        groups[g] = {
            "kernels": kernels,
            "fetch_KiB_per_step": tot["FETCH_SIZE"],
            "write_KiB_per_step": tot["WRITE_SIZE"],
            "hbm_bytes_per_step": tot["FETCH_SIZE"] * 1024 * scale["FETCH_SIZE"]
            + tot["WRITE_SIZE"] * 1024 * scale["WRITE_SIZE"],
        }
        # L2 counters of a further pass, when one was given: hit rate and
        # the 128-byte line reads L2 sent to memory (TCC_EA0_RDREQ), of them
        # those addressed to DRAM; rocprofv3 on gfx950 has no counter of the
        # memory-side cache (MALL), so DRAM-addressed reads are an upper
        # bound on the reads HBM served.
        l2 = {}
        for ctr in ("TCC_HIT_sum", "TCC_MISS_sum", "TCC_EA0_RDREQ_sum", "TCC_EA0_RDREQ_DRAM_sum"):
            vals = [float(np.mean(v)) * len(v) / steps_run for n, v in per.get(ctr, {}).items()
                    if any(p in n for p in pats)]
            if vals:
                l2[ctr + "_per_step"] = float(sum(vals))
        if "TCC_HIT_sum_per_step" in l2 and "TCC_MISS_sum_per_step" in l2:
            hm = l2["TCC_HIT_sum_per_step"] + l2["TCC_MISS_sum_per_step"]
            l2["l2_hit_rate"] = l2["TCC_HIT_sum_per_step"] / hm if hm else None
        if l2:
            groups[g]["l2"] = l2
    res = {"config": config, "source_stamp": source_stamp(), "steps_run": steps_run, "copy_kernel": cname,
           "copy_bytes": COPY_BYTES,
           "copy_FETCH_KiB": f_kib,
           "copy_WRITE_KiB": w_kib, "scale": scale, "groups": groups}
    Path(out_path).write_text(json.dumps(res, indent=1) + "\n")
    print(json.dumps(res, indent=1))


def summarize_trace(dirs, out_path, title, command):
    """Markdown table of per-kernel durations from rocprofv3 --kernel-trace."""

    agg = {}
    for name, dur in _rocpd_rows(dirs, "select name, duration from kernels"):
        agg.setdefault(name.replace("void ", "").split("(")[0], []).append(float(dur))
    # The library's kernels are the steps; torch's (random table init, fills)
    # run while the bench sets up, outside the timed steps.
    ours = {k: v for k, v in agg.items() if k.startswith("mdl::")}
    setup = {k: v for k, v in agg.items() if not k.startswith("mdl::")}
    total = sum(sum(v) for v in ours.values())
    lines = [f"# {title}", "", "```", command, "```", "",
             "Library kernels (share of their summed time):", "",
             "| kernel | calls | avg us | total ms | share |", "|---|---:|---:|---:|---:|"]
    for k, v in sorted(ours.items(), key=lambda kv: -sum(kv[1])):
        lines.append(f"| `{k}` | {len(v)} | {np.mean(v) / 1e3:.1f} | {sum(v) / 1e6:.2f} | {100 * sum(v) / total:.1f}% |")
    lines += ["", "Set-up kernels (torch: table init, fills; not in the timed steps):", "",
              "| kernel | calls | avg us | total ms |", "|---|---:|---:|---:|"]
    for k, v in sorted(setup.items(), key=lambda kv: -sum(kv[1])):
        lines.append(f"| `{k[:80]}` | {len(v)} | {np.mean(v) / 1e3:.1f} | {sum(v) / 1e6:.2f} |")
    Path(out_path).write_text("\n".join(lines) + "\n")
    print("\n".join(lines))


def source_stamp() -> str:
    """Hash of the library's sources (kernels, header, build flags): a
    counter summary is only valid for the build it was measured on."""

    import hashlib

    h = hashlib.sha256()
    csrc = ROOT / "mdl_amd" / "csrc"
    for p in sorted(list(csrc.glob("*.hip")) + list(csrc.glob("*.cuh")) + [csrc / "Makefile",
                    ROOT / "include" / "mdl_hip.h"]):
        h.update(p.name.encode())
        h.update(p.read_bytes())
    return h.hexdigest()[:16]


def load_traffic(config: str):
    """(summary, reason): the committed counter summary of ``config`` when it
    was measured on these library sources, else (None, why not)."""

    p = ROOT / "profiles" / f"{config}_traffic.json"
    if not p.exists():
        return None, f"no profiles/{config}_traffic.json"
    try:
        tr = json.loads(p.read_text())
    except (OSError, ValueError):
        return None, f"profiles/{config}_traffic.json unreadable"
    stamp = source_stamp()
    if tr.get("source_stamp") != stamp:
        return None, (f"profiles/{config}_traffic.json was measured on library sources "
                      f"{tr.get('source_stamp')}, not these ({stamp}): not used")
    return tr, ""


# ------------------------------------------------------------------- main --


def measure(name: str, args, torch, device, *, with_aux: bool = False) -> dict:
    """Time one config: ``args.warmup`` untimed steps, ``args.steps`` timed
    between device synchronisations (a different batch bound every step),
    then the same number of steps with HIP events around the forward and the
    apply.  Returns the fields of the bench line for that config."""

    wl = WORKLOADS[name]()
    print(f"[bench] workload {wl.name}: {len(wl.features)} features, {len(wl.rows)} tables, "
          f"{sum(wl.rows):.3e} rows, batch {wl.batch}, {wl.dtype}", file=sys.stderr, flush=True)
    rng = np.random.default_rng(99)
    batches = [draw_batch(rng, wl) for _ in range(args.batches)]
    alg = [algorithmic_bytes(wl, ids, lengths) for ids, lengths in batches]
    print(f"[bench] {wl.name}: drew {args.batches} batches; {alg[0]['n_ids']} ids/step, "
          f"{alg[0]['unique_rows']} distinct rows", file=sys.stderr, flush=True)
    if wl.kind == "sequence":
        dev = SequenceDeviceStep(wl, batches, device)
    else:
        dev = DeviceStep(wl, batches, device, layout=args.layout)
    torch.cuda.synchronize()
    print(f"[bench] {wl.name}: tables initialised", file=sys.stderr, flush=True)
    if args.calibrate_copy:
        # a plain streaming kernel of known traffic: read 1 GiB, write 1 GiB
        src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device=device)
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst
    for i in range(args.warmup):
        dev.step(i)
    torch.cuda.synchronize()
    if args.graph:
        # each batch's step as one HIP graph (recorded after the eager warmup
        # steps loaded the kernels); the timed steps replay them
        dev.capture()
        torch.cuda.synchronize()
        for i in range(len(dev.batches)):
            dev.step(args.warmup + i)
        torch.cuda.synchronize()
    if int(dev.err.item()):
        raise RuntimeError("synthetic ids out of range")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        dev.step(args.warmup + i)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms = elapsed * 1e3 / args.steps
    used = [alg[(args.warmup + i) % len(alg)] for i in range(args.steps)]
    n_ids = float(np.mean([a["n_ids"] for a in used]))
    b_alg = float(np.mean([a["B_alg"] for a in used]))
    # Per-kernel durations: HIP events around each call on the launch stream,
    # in separate (untimed) steps so the event records do not touch the step time.
    timers = {"forward": EventTimer(torch), "apply": EventTimer(torch)}
    for i in range(args.steps):
        dev.step(args.warmup + args.steps + i, timers)
    torch.cuda.synchronize()
    if int(dev.err.item()):
        raise RuntimeError("synthetic ids out of range")
    esz = 4 if wl.dtype == "fp32" else 2
    nb = float(np.mean([sum(len(ln) for ln in b[1] if ln is not None) for b in batches]))
    kernels = {}
    if wl.kind == "sequence":
        _, _, pad = wl.seq_len
        nf = len(wl.features)
        d = wl.dims[0]
        # ids of the valid positions + lengths read, distinct rows, padded
        # window + mask, sort keys/payloads (packed: one per looked-up id)
        fwd_bytes = float(np.mean([8 * a["n_ids"] + 8 * nf * wl.batch + a["fwd_unique_row_bytes"]
                                   + nf * wl.batch * pad * (d * esz + 1) + 8 * a["n_ids"] for a in used]))
        # sorted keys/payloads, gradient rows at valid positions, rows read+written, state
        apply_bytes = float(np.mean([8 * a["n_ids"] + a["n_ids"] * d * esz
                                     + 2 * a["fwd_unique_row_bytes"] + 8 * a["unique_rows"] for a in used]))
    else:
        fwd_bytes = float(np.mean([16 * a["n_ids"] + 8 * (nb + 1) + a["fwd_unique_row_bytes"]
                                   + wl.batch * a["sum_dim"] * esz + 4 * nb for a in used]))
        apply_bytes = float(np.mean([8 * a["n_ids"] + wl.batch * a["sum_dim"] * esz
                                     + 2 * a["fwd_unique_row_bytes"] + 8 * a["unique_rows"] + 4 * nb for a in used]))
    fwd_label = ("sequence_kernel + sequence_keys_kernel per feature (window gather, mask, sort keys)"
                 if wl.kind == "sequence" else "forward_kernel (grouped lookup + pooling + sort-key emission)")
    for kname, nbytes, label in (
        ("forward", fwd_bytes, fwd_label),
        ("apply", apply_bytes, "bwd_reduce_kernel + fix-up (segment reduction + row-wise Adagrad)"),
    ):
        kms = timers[kname].median_ms()
        kernels[kname] = {"kernel": label, "ms": kms, "alg_bytes_per_launch": nbytes,
                          "achieved_gbps": nbytes / (kms * 1e-3) / 1e9}
    dom_name = max(kernels, key=lambda k: kernels[k]["ms"])
    dom = kernels[dom_name]
    traffic = None
    tr, why = load_traffic(wl.name)
    if tr is not None:
        # counter bytes of each launch group per looked-up row (the
        # per-row traffic figure of the measurement plan), with its L2 hit rate
        for kname, g in tr.get("groups", {}).items():
            rec = kernels.setdefault(kname, {"kernel": kname})
            rec["counter_bytes"] = g["hbm_bytes_per_step"]
            rec["counter_bytes_per_looked_up_row"] = g["hbm_bytes_per_step"] / max(n_ids, 1.0)
            if "l2" in g and g["l2"].get("l2_hit_rate") is not None:
                rec["l2_hit_rate"] = g["l2"]["l2_hit_rate"]
    if tr is not None and "hbm_bytes_per_step" in tr.get("groups", {}).get(dom_name, {}):
        traffic = tr["groups"][dom_name]["hbm_bytes_per_step"]
        dom["traffic_source"] = (f"profiles/{wl.name}_traffic.json (rocprofv3 FETCH_SIZE/WRITE_SIZE, copy-calibrated; "
                                 f"library sources {tr['source_stamp']})")
    else:
        dom["traffic_source"] = why
    out = {
        "workload": f"{wl.name}: {len(wl.features)} features, batch {wl.batch}, "
                    f"{sum(wl.rows):.3e} table rows, {wl.dtype} tables, fused fwd+bwd+row-wise Adagrad",
        "value": n_ids / (ms * 1e-3),
        "ms_per_step": ms,
        "global_batch": wl.batch,
        "ids_per_step": n_ids,
        "distinct_rows_per_step": float(np.mean([a["unique_rows"] for a in used])),
        "dtype": "f32" if wl.dtype == "fp32" else "bf16-storage/f32-accumulate",
        "hbm_gbps_achieved": b_alg / (ms * 1e-3) / 1e9,
        "roofline_fraction_step": b_alg / (ms * 1e-3) / 1e9 / PEAK_HBM_GBPS,
        # every launch group's measured traffic over the step time: how busy
        # HBM is over the whole step in the whole lines it moves
        "traffic_fraction_step": (None if tr is None else sum(g["hbm_bytes_per_step"] for g in tr["groups"].values())
                                  / (ms * 1e-3) / 1e9 / PEAK_HBM_GBPS),
        "B_alg_bytes_per_step": b_alg,
        "roofline": {
            "kernel": dom["kernel"],
            "bound": "hbm",
            "achieved": dom["achieved_gbps"],
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": dom["achieved_gbps"] / PEAK_HBM_GBPS,
            "traffic": traffic,
            # the measured traffic over the same time against the same peak:
            # how busy HBM is in the bytes it moves (whole lines), where frac
            # counts only the bytes the algorithm needs
            "traffic_frac": None if traffic is None else traffic / (dom["ms"] * 1e-3) / 1e9 / PEAK_HBM_GBPS,
            "kernel_ms": dom["ms"],
            "alg_bytes_per_launch": dom["alg_bytes_per_launch"],
        },
        "kernels": kernels,
        "batches": args.batches,
        "aux": None,
    }
    if with_aux and wl.kind != "sequence":
        # after every timed number above, so the extra steps change none of them
        out["aux"] = aux_measurements(torch, dev, wl, n_ids, args.steps, device, batches)
    del dev
    # Tables held in reference cycles (autograd records, optimizer state of
    # the drop-in loop) go now, before the next config allocates its own.
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    print(f"[bench] {wl.name}: done; {torch.cuda.memory_allocated(device) / 2**30:.1f} GiB still allocated",
          file=sys.stderr, flush=True)
    out["_wl"] = wl
    out["_batch0"] = batches[0]
    return out


def ceilings(torch, device) -> dict:
    """What this MI355X sustains on the access patterns of the path, measured
    with the product's own kernels and torch's copy: device copies of 256 MiB
    to 4 GiB, the library's streaming bucketize (8 bytes read, 8 written per
    id) on 32 M to 512 M ids, and gathers of 16 M uniformly random rows (no reuse) of
    16..512 bytes from one 64 GiB-class table through ``mdl_forward``
    (unpooled), each timed with HIP events over 10 launches behind a spin
    kernel.  The gather's rows/s at small rows is the request ceiling the
    step's kernels are compared with; the same gather over tables of 1 to 192
    GiB shows whether address translation bounds it."""

    from mdl_amd import ops

    out = {}
    reps = 10

    def timed(fn):
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(20_000_000)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    copies = []
    for nbytes in (1 << 28, 1 << 30, 1 << 32):
        src = torch.empty(nbytes // 4, dtype=torch.float32, device=device).fill_(1.0)
        dst = torch.empty_like(src)
        ms = timed(lambda: dst.copy_(src))
        copies.append({"bytes_read": nbytes, "ms": ms, "gbps": 2.0 * nbytes / (ms * 1e-3) / 1e9})
        del src, dst
    out["torch_copy"] = copies
    # the library's own streaming kernel: mdl_bucketize reads 8 and writes 8
    # bytes per id, coalesced
    streams = []
    for n in (1 << 25, 1 << 27, 1 << 29):
        raw = torch.randint(1, 1 << 62, (n,), dtype=torch.int64, device=device)
        ids = torch.empty_like(raw)
        ms = timed(lambda: ops.bucketize(raw, 1 << 20, validate_nonzero=False))
        streams.append({"ids": n, "bytes": 16.0 * n, "ms": ms, "gbps": 16.0 * n / (ms * 1e-3) / 1e9})
        del raw, ids
        gc.collect()
        torch.cuda.empty_cache()
    out["stream_bucketize"] = streams
    torch.cuda.empty_cache()
    n = 1 << 24
    gen = torch.Generator(device=device)
    gen.manual_seed(5)
    rows_out = []
    for row_bytes in (16, 32, 64, 128, 256, 512):
        dim = row_bytes // 4
        rows = (48 << 30) // row_bytes  # 48 GiB of rows: far beyond L2 and the memory-side cache
        table = torch.empty((rows, dim), dtype=torch.float32, device=device)
        ids = torch.randint(0, rows, (n,), dtype=torch.int64, device=device, generator=gen)
        plan = ops.GroupPlan()
        plan.add_feature(table, pooling="none")
        outbuf = torch.empty((n, dim), dtype=torch.float32, device=device)
        ms = timed(lambda: ops.grouped_forward(plan, [ids], [None], with_backward=False, outputs=[outbuf]))
        lines = -(-row_bytes // 128)  # 128-byte lines a row read costs
        rows_out.append({
            "row_bytes": row_bytes, "rows": n, "ms": ms, "rows_per_s": n / (ms * 1e-3),
            "row_read_gbps": n * row_bytes / (ms * 1e-3) / 1e9,
            "line_reads_per_s": n * lines / (ms * 1e-3),
            "write_gbps": n * row_bytes / (ms * 1e-3) / 1e9,
        })
        del table, ids, outbuf, plan
        gc.collect()
        torch.cuda.empty_cache()
    out["random_row_gather"] = rows_out
    # Address translation: the same gather of 16 M uniformly random rows from
    # tables of 1 GiB to 192 GiB (c4's 8 large bf16 tables hold 192 GB).  A
    # rate that holds as the footprint grows past what the TLBs map says the
    # gathers are bound by memory requests, not by page walks.
    footprint = []
    for row_bytes in (64, 128):
        dim = row_bytes // 4
        for gib in (1, 16, 64, 192):
            rows = (gib << 30) // row_bytes
            table = torch.empty((rows, dim), dtype=torch.float32, device=device)
            ids = torch.randint(0, rows, (n,), dtype=torch.int64, device=device, generator=gen)
            plan = ops.GroupPlan()
            plan.add_feature(table, pooling="none")
            outbuf = torch.empty((n, dim), dtype=torch.float32, device=device)
            ms = timed(lambda: ops.grouped_forward(plan, [ids], [None], with_backward=False, outputs=[outbuf]))
            footprint.append({"row_bytes": row_bytes, "table_gib": gib, "rows": n, "ms": ms,
                              "rows_per_s": n / (ms * 1e-3)})
            del table, ids, outbuf, plan
            gc.collect()
            torch.cuda.empty_cache()
    out["random_row_footprint"] = footprint
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="c1", choices=sorted(WORKLOADS))
    ap.add_argument("--batches", type=int, default=3, help="distinct synthetic batches, one bound per step in turn")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="only the headline config (by default every other config is measured after it)")
    ap.add_argument("--graph", action="store_true",
                    help="replay one HIP graph per batch instead of launching each step's kernels from the host "
                         "(measured: no faster at c0, c1 or c4 -- the host keeps ahead of the GPU)")
    ap.add_argument("--no-aux", action="store_true",
                    help="skip the clipped-step and bucketing measurements (off with --calibrate-copy)")
    ap.add_argument("--cpu-steps", type=int, default=5, help="timed steps of the CPU baseline (after 2 warmup)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run three plain 1 GiB device copies (counter calibration for rocprofv3 --pmc runs)")
    ap.add_argument("--summarize-pmc", nargs="+", metavar="DIR",
                    help="summarise rocprofv3 --pmc databases into --pmc-out and exit (no GPU); give the "
                         "--steps/--warmup of the profiled run")
    ap.add_argument("--pmc-out", default=None)
    ap.add_argument("--summarize-trace", nargs="+", metavar="DIR",
                    help="summarise rocprofv3 --kernel-trace databases into --trace-out and exit (no GPU)")
    ap.add_argument("--trace-out", default=None)
    ap.add_argument("--trace-command", default="")
    ap.add_argument("--ceilings", action="store_true",
                    help="measure the copy and random-row-gather ceilings of this GPU and exit (one JSON line)")
    ap.add_argument("--layout", choices=["slot", "feature"], default="slot",
                    help="pooled outputs and their gradients: one [B, sum(dim)] token-slot buffer, or one [B, dim] "
                         "tensor per feature")
    args = ap.parse_args()
    if args.summarize_pmc:
        # the profiled run made warmup + steps timed + steps per-kernel-timed step() calls;
        # pass the same --steps/--warmup here
        summarize_pmc(args.summarize_pmc, args.pmc_out or str(ROOT / "profiles" / f"{args.config}_traffic.json"),
                      args.config, args.warmup + 2 * args.steps)
        return 0
    if args.summarize_trace:
        summarize_trace(args.summarize_trace, args.trace_out or "/dev/stdout",
                        f"{args.config}: rocprofv3 kernel trace", args.trace_command)
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported in this build "
              "(the path is single-GPU; multi-GPU sharding is a design note, not a measured run)",
              file=sys.stderr)
        return 2

    import torch

    device = torch.device("cuda:0")
    if args.ceilings:
        print(json.dumps(ceilings(torch, device)), flush=True)
        return 0
    head = measure(args.config, args, torch, device,
                   with_aux=not args.no_aux and not args.calibrate_copy)
    wl = head.pop("_wl")
    batch0 = head.pop("_batch0")
    result = {
        "metric": METRIC,
        "value": head["value"],
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": head["dtype"],
        "data": "synthetic (seeded Zipf ids, random-init tables); a different batch bound every step",
        "config": {
            "workload": head["workload"],
            "global_batch": head["global_batch"],
            "ids_per_step": head["ids_per_step"],
            "distinct_rows_per_step": head["distinct_rows_per_step"],
            "parallelism": "single GPU",
            "launch": "one HIP graph per batch (captured step)" if args.graph else "eager",
            "batches": args.batches,
        },
        "hbm_gbps_achieved": head["hbm_gbps_achieved"],
        "roofline_fraction_step": head["roofline_fraction_step"],
        "traffic_fraction_step": head["traffic_fraction_step"],
        "B_alg_bytes_per_step": head["B_alg_bytes_per_step"],
        "roofline": head["roofline"],
        "kernels": head["kernels"],
        "aux": head["aux"],
        "cpu_baseline": None,
        "configs": {},
    }
    # Every GPU timing first, the CPU restatements last: a CPU baseline runs
    # all host threads over up to 160 GB of host tables, and the short steps
    # of the small configs are paced by the host's launches.
    cpu_runs = []
    if not args.no_cpu_baseline and not args.calibrate_copy:
        cpu_runs.append((result, wl, batch0))
    if not args.no_configs and not args.calibrate_copy:
        for name in ("c0", "c3", "c4", "c2"):
            if name == args.config:
                continue
            m = measure(name, args, torch, device)
            mwl = m.pop("_wl")
            mb = m.pop("_batch0")
            m.pop("aux")
            if name == "c0" and not args.no_cpu_baseline:
                cpu_runs.append((m, mwl, mb))  # the CPU-runnable plumbing config, at full size
            result["configs"][name] = m
            print(f"[bench] {name}: {m['ms_per_step']:.3f} ms/step, {m['value']:.3e} rows/s, "
                  f"step {m['roofline_fraction_step']:.3f} of HBM peak", file=sys.stderr, flush=True)
    for entry, cwl, cbatch in cpu_runs:
        print(f"[bench] timing the CPU restatement on {cwl.name}", file=sys.stderr, flush=True)
        entry["cpu_baseline"] = cpu_baseline(cwl, cbatch, steps=args.cpu_steps)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
