"""One fused sparse step per batch over a fixed feature layout.

``SparseStep`` binds a feature layout (:class:`mdl_amd.ops.GroupPlan`) to its
outputs, upstream gradients and scratch, and builds every descriptor, chunk
table and workspace once.  A step is then launches only -- no host work,
allocation or synchronisation:

    lengths -> offsets scan, grouped lookup + pooling (+ sort keys),
    radix sort, segment reduction + row-wise Adagrad.

Any batch of the layout (same features and batch size; bag lengths free)
runs on the same object: :meth:`SparseStep.bind` points the step at the
batch's packed ids and bag lengths, the offsets scan places every feature's
ids on the device, and the sort and reduce take the batch's id count from
the scan's last offset.  This is what the reference encoder does for every
training batch (src/model.py:3782-3890), with the pooled outputs written
straight into caller-given views such as the RankMixer token-slot buffer
``[B, sum(dim)]``.
"""

from __future__ import annotations

from typing import Sequence

import numpy as np
import torch
from torch import Tensor

from . import ops
from ._lib import CHUNK_DTYPE, FEATURE_DTYPE, MDL_FLAG_IDS_FROM_OFFSETS, MDL_POOL_NONE, check, lib

# Descriptor bound of a feature whose ids the offsets place: the call's id
# count clamps the range anyway.
_NO_BOUND = 1 << 62


def _capture(device: torch.device, fn) -> "torch.cuda.CUDAGraph":
    """fn's launches recorded on a side stream of default priority."""

    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(device=device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.graph(graph, stream=side):
        fn()
    torch.cuda.current_stream(device).wait_stream(side)
    return graph


def _as_ids(t: Tensor) -> Tensor:
    if t.dtype != torch.int64:
        raise TypeError("sharded embedding indices must be torch.long")
    return t.contiguous()


class _KeyGroup:
    """Device state of one key group of a step: its forward descriptors and
    chunks, sort keys and payloads, backward descriptors, tables and
    workspace."""

    F: int
    feats_fwd_dev: Tensor
    chunks_dev: Tensor
    n_chunks: int
    fwd_classes: int
    feats_bwd: np.ndarray
    feats_bwd_dev: Tensor
    tables: np.ndarray
    tables_dev: Tensor
    bwd_classes: int
    keys: Tensor
    payload: Tensor
    ws: Tensor


class SparseStep:
    """Fused lookup/pooling + backward + row-wise Adagrad for one layout.

    ``packed_ids``: every feature's ids back to back (device int64);
    ``lengths``: every pooled feature's bag lengths back to back, with one
    pseudo-length (its id count) per unpooled feature, in feature order --
    None when no feature is pooled; ``id_counts`` / ``bag_counts``: per
    feature, for this first batch (they size the chunks; bag counts are the
    batch size of each pooled feature and stay fixed, and so does the id count
    of an unpooled feature, one per output row).  ``capacity`` bounds the ids
    of any batch bound later (default: this batch's).  Outputs and gradients
    are 2-D row views (e.g. column slices of one ``[B, sum(dim)]`` buffer).

    Gradient accumulation (src/train.py:7007-7067, :5388-5396): with
    ``micro_batches=k``, ``outputs`` and ``grads`` are k lists of views, one
    per micro-batch; ``forward(micro_batch=m)`` looks up micro-batch m (bound
    with :meth:`bind` before it) into its outputs and its own region of the
    sort keys, and one ``sort()`` + ``apply()`` then reduces the gradients of
    all k micro-batches together -- the sum of their sparse gradients, each
    row updated once -- instead of coalescing an accumulated COO gradient.
    """

    def __init__(
        self,
        plan: ops.GroupPlan,
        packed_ids: Tensor,
        lengths: Tensor | None,
        id_counts: Sequence[int],
        bag_counts: Sequence[int],
        outputs: Sequence[Tensor],
        grads: Sequence[Tensor],
        *,
        error_count: Tensor | None = None,
        capacity: int | None = None,
        micro_batches: int = 1,
    ) -> None:
        for t in plan.tables:
            if t.state is None:
                raise RuntimeError("every table needs a row-wise Adagrad accumulator")
        self.k = int(micro_batches)
        if self.k < 1:
            raise ValueError("micro_batches must be positive")
        self._looked_up: set[int] = set()  # micro-batches forwarded since the last sort
        if self.k == 1:
            outputs, grads = [outputs], [grads]
        elif len(outputs) != self.k or len(grads) != self.k:
            raise ValueError("one list of outputs and one of gradients per micro-batch")
        self.plan = plan
        self.device = packed_ids.device
        self.ids = _as_ids(packed_ids)
        self.capacity = max(int(self.ids.numel()) if capacity is None else int(capacity), int(self.ids.numel()))
        pooled_any = any(s.pooling != MDL_POOL_NONE for s in plan.features)
        self.dynamic = pooled_any
        self.lengths = None
        self.offsets = None
        if pooled_any:
            if lengths is None:
                raise ValueError("pooled features need bag lengths")
            self.lengths = lengths.to(torch.int64).contiguous()
            nl = int(self.lengths.numel())
            self.offsets = torch.empty(nl + 1, dtype=torch.int64, device=self.device)
            self.scan_ws = ops._workspace(lib().mdl_offsets_workspace_bytes(nl), self.device)
        self.error_count = (
            error_count if error_count is not None else torch.zeros(1, dtype=torch.int32, device=self.device)
        )
        out_ptrs = [o.data_ptr() for o in outputs[0]]
        out_strides = [o.stride(0) if o.ndim == 2 else int(o.size(-1)) for o in outputs[0]]
        feats = ops.build_features(plan, id_counts, bag_counts, out_ptrs, out_strides)
        groups = plan.groups
        # Chunks of each key group, planned on this batch's id counts (a
        # group's chunks number its features from the group's first).
        chunks = []
        for g in groups:
            sub = np.ascontiguousarray(feats[g.lo: g.hi])
            target = ops.forward_target_ids(sub)
            nc = lib().mdl_plan_chunks(sub.ctypes.data, len(sub), target, None, 0)
            if nc < 0:
                check(int(nc), "mdl_plan_chunks")
            ch = np.zeros(max(nc, 1), dtype=CHUNK_DTYPE)
            lib().mdl_plan_chunks(sub.ctypes.data, len(sub), target, ch.ctypes.data, nc)
            chunks.append((ch, int(nc)))
        first_ids = feats["ids_begin"].copy()
        if self.dynamic:
            # The offsets of each call place every feature's ids.
            feats["flags"] |= MDL_FLAG_IDS_FROM_OFFSETS
            feats["ids_begin"] = 0
            feats["num_ids"] = _NO_BOUND
        total_rows = int(
            np.where(feats["pooling"] != MDL_POOL_NONE, feats["num_bags"], np.asarray(id_counts)).sum()
        )
        self.rows_per_batch = max(total_rows, 1)
        if self.rows_per_batch * self.k >= 1 << 32:
            raise ValueError("the micro-batches' output rows exceed the 32-bit gradient-row payload")
        # Micro-batch m: its forward descriptors (its outputs, payloads and
        # bag counts shifted by m rows-per-batch) and its backward ones (its
        # gradients).
        fwd, bwd = [], []
        self._grads = []
        for m in range(self.k):
            if [o.stride(0) if o.ndim == 2 else int(o.size(-1)) for o in outputs[m]] != out_strides:
                raise ValueError("every micro-batch's outputs need the row strides of the first's")
            fm = feats.copy()
            fm["out"] = [o.data_ptr() for o in outputs[m]]
            fm["payload_base"] += m * self.rows_per_batch
            fwd.append(fm)
            res = ops.ForwardResult(
                plan=plan, device=self.device, ids=self.ids, offsets=None, outputs=list(outputs[m]),
                feats=fm, keys=None, payload=None, bag_count=None, error_count=self.error_count,
            )
            fb, keep = ops._attach_grads(res, grads[m])
            bwd.append(fb)
            self._grads += keep
        self.feats_fwd = fwd[0]
        self.bag_count = (
            torch.empty(self.rows_per_batch * self.k, dtype=torch.float32, device=self.device) if pooled_any else None
        )
        cap = max(self.capacity, 1)
        n_sort = self._n()
        self.groups = []
        for g, (ch, nc) in zip(groups, chunks):
            gs = _KeyGroup()
            gs.F = g.hi - g.lo
            # all micro-batches' descriptors of the group's features, micro-batch 0 first
            f_fwd = np.concatenate([fm[g.lo: g.hi] for fm in fwd])
            gs.feats_bwd = np.concatenate([fb[g.lo: g.hi] for fb in bwd])
            gs.tables = ops._tables_array(g.plan, np.ascontiguousarray(bwd[0][g.lo: g.hi]))
            if self.k > 1:
                # a table read by k copies of its feature: the reduce finds each
                # payload's feature by search instead of the one-feature path
                gs.tables["feature"] = -1
            gs.fwd_classes = ops.feature_classes(np.ascontiguousarray(fwd[0][g.lo: g.hi]))
            gs.bwd_classes = ops.table_classes(gs.tables)
            gs.feats_fwd_dev = ops.upload(f_fwd, self.device)
            gs.chunks_dev = ops.upload(ch, self.device)
            gs.n_chunks = nc
            gs.feats_bwd_dev = ops.upload(gs.feats_bwd, self.device)
            gs.tables_dev = ops.upload(gs.tables, self.device)
            gs.keys = torch.empty(cap * self.k, dtype=torch.int32, device=self.device)
            gs.payload = torch.empty(cap * self.k, dtype=torch.int32, device=self.device)
            gs.ws = ops._workspace(
                lib().mdl_backward_workspace_bytes(n_sort, len(gs.tables), plan.max_dim), self.device
            )
            self.groups.append(gs)
        G = len(self.groups)
        if G > 1:
            # Each group's ids are one stretch of the packed ids: its first
            # position (the key origin of its forward) and its id count, on
            # the device -- from the offsets scan when bag lengths place them.
            lo = np.array([g.lo for g in groups], dtype=np.int64)
            hi = np.array([g.hi for g in groups], dtype=np.int64)
            if self.dynamic:
                bags = np.append(feats["bag_base"], int(self.lengths.numel()))
                self._gidx = ops.upload(np.concatenate([bags[lo], bags[hi]]), self.device).view(torch.int64)
                self._gsel = torch.empty(2 * G, dtype=torch.int64, device=self.device)
                self._gcount = torch.empty(G, dtype=torch.int64, device=self.device)
            else:
                ends = np.append(first_ids, int(self.ids.numel()))
                self._gsel = ops.upload(np.concatenate([ends[lo], ends[hi]]), self.device).view(torch.int64)
                self._gcount = ops.upload(ends[hi] - ends[lo], self.device).view(torch.int64)
        if self.k > 1:
            self._positions = torch.arange(cap, dtype=torch.int64, device=self.device)
            sentinel = int(plan.sentinel)
            self._sentinel = sentinel - (1 << 32) if sentinel >= (1 << 31) else sentinel
        self._empty_ids = torch.zeros(1, dtype=torch.int64, device=self.device)
        self.sumsq = torch.zeros(G, dtype=torch.float32, device=self.device)
        self.norm = torch.zeros(1, dtype=torch.float32, device=self.device)
        self.coef = torch.ones(1, dtype=torch.float32, device=self.device)
        # what the update mutates, named in the ops' schemas
        self._weights = [t.weight for t in plan.tables]
        self._states = [t.state for t in plan.tables]
        self._outs = [o for outs in outputs for o in outs]

    # ----------------------------------------------------------- batches --

    def bind(self, packed_ids: Tensor, lengths: Tensor | None = None) -> None:
        """Point the next steps at another batch of this layout (no copy, no
        sync).  A captured graph keeps the buffers it was recorded with: to
        replay it on a new batch, copy the batch into ``self.ids`` /
        ``self.lengths`` instead."""

        ids = _as_ids(packed_ids)
        if ids.device != self.device:
            raise ValueError("ids must live on the step's device")
        if int(ids.numel()) > self.capacity:
            raise ValueError(f"batch of {ids.numel()} ids exceeds the step's capacity of {self.capacity}")
        if not self.dynamic:
            if int(ids.numel()) != int(self.ids.numel()):
                raise ValueError("a layout without pooled features keeps its id count")
        elif lengths is not None:
            ln = lengths if lengths.dtype == torch.int64 else lengths.to(torch.int64)
            ln = ln.contiguous()
            if ln.shape != self.lengths.shape or ln.device != self.device:
                raise ValueError("bag lengths must keep the layout's shape and device")
            self.lengths = ln
        self.ids = ids

    @property
    def count(self) -> Tensor | None:
        """Device int64 [1]: ids of the bound batch (the scan's last offset)."""

        return None if self.offsets is None else self.offsets[-1:]

    def _stream(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    def _count(self, g: int) -> tuple[Tensor | None, int]:
        """Group g's entry count on the device: (tensor, element offset);
        (None, 0) when the sort takes all of its capacity."""

        if len(self.groups) > 1:
            return self._gcount, g
        return (None, 0) if self.offsets is None else (self.offsets, int(self.offsets.numel()) - 1)

    def _n(self) -> int:
        if self.k > 1:
            return max(self.capacity, 1) * self.k
        return self.capacity if self.dynamic or len(self.plan.groups) > 1 else int(self.ids.numel())

    # ------------------------------------------------------------- steps --

    def forward(self, micro_batch: int = 0) -> None:
        """Offsets scan + grouped lookup/pooling (+ backward sort keys) of the
        bound batch, as micro-batch ``micro_batch`` of an accumulated step."""

        m = int(micro_batch)
        if not 0 <= m < self.k:
            raise ValueError(f"micro_batch must be in [0, {self.k})")
        self._looked_up.add(m)
        s = self._stream()
        if self.offsets is not None:
            check(
                lib().mdl_lengths_to_offsets(
                    self.lengths.data_ptr(), self.lengths.numel(), self.offsets.data_ptr(),
                    self.scan_ws.data_ptr(), self.scan_ws.numel(), s,
                ),
                "mdl_lengths_to_offsets",
            )
        G = len(self.groups)
        if G > 1 and self.dynamic:
            torch.index_select(self.offsets, 0, self._gidx, out=self._gsel)
            torch.sub(self._gsel[G:], self._gsel[:G], out=self._gcount)
        ids = self.ids if self.ids.numel() else self._empty_ids  # any valid address; nothing is read
        region = m * max(self.capacity, 1)
        for g, gs in enumerate(self.groups):
            torch.ops.mdl_hip.packed_forward_(
                gs.feats_fwd_dev, m * gs.F, gs.F, gs.chunks_dev, gs.n_chunks, ids, int(self.ids.numel()),
                self.offsets, gs.keys, gs.payload, region, None if G == 1 else self._gsel, g, self.plan.sentinel,
                self.bag_count, self.error_count, self._outs, gs.fwd_classes,
            )
            if self.k > 1:
                # entries of the region past this micro-batch's ids sort last
                # and reduce nowhere
                if G > 1:
                    live = self._gcount[g]
                else:
                    live = self.offsets[-1] if self.offsets is not None else int(self.ids.numel())
                gs.keys[region: region + max(self.capacity, 1)].masked_fill_(self._positions >= live, self._sentinel)

    def _check_micro_batches(self) -> None:
        # Every region of the keys must hold this step's lookup: a region left
        # from an earlier step would apply its gradients a second time.
        if self.k > 1:
            if len(self._looked_up) != self.k:
                missing = sorted(set(range(self.k)) - self._looked_up)
                raise RuntimeError(f"micro-batches {missing} were not looked up since the last sort")
            self._looked_up.clear()

    def sort(self) -> None:
        """Radix sort of the (row, gradient-row) pairs + chunk plan."""

        self._check_micro_batches()
        for g, gs in enumerate(self.groups):
            count, at = self._count(g) if self.k == 1 else (None, 0)
            torch.ops.mdl_hip.backward_sort_(gs.tables_dev, len(gs.tables), gs.keys, gs.payload, self._n(), count, at,
                                             self.plan.max_dim, self.plan.key_bits, gs.ws)

    def apply(self, lr: float, eps: float, grad_scale: Tensor | None = None) -> None:
        """Segment reduction of duplicate rows + fused row-wise Adagrad
        (gradients times ``grad_scale``, a device fp32 [1], when given)."""

        for gs in self.groups:
            torch.ops.mdl_hip.backward_apply_(
                self._weights, self._states, gs.feats_bwd_dev, len(gs.feats_bwd), gs.tables_dev, len(gs.tables),
                gs.keys, gs.payload, self._n(), self.bag_count, grad_scale, gs.ws, self.plan.max_dim,
                self.plan.key_bits, gs.bwd_classes, float(lr), float(eps),
            )

    def clip(self, max_norm: float) -> tuple[Tensor, Tensor]:
        """After sort(): (pre-clip global norm, clip coefficient), on device.

        The norm is that of the coalesced gradient of every table, as the
        trainer's sparse clip computes it (src/train.py:5788-5826)."""

        for g, gs in enumerate(self.groups):
            torch.ops.mdl_hip.backward_sumsq_(
                gs.feats_bwd_dev, len(gs.feats_bwd), gs.tables_dev, len(gs.tables), gs.keys, gs.payload, self._n(),
                self.bag_count, self.sumsq, g, gs.ws, self.plan.max_dim, self.plan.key_bits, gs.bwd_classes,
            )
        torch.ops.mdl_hip.clip_coefficient_(self.sumsq, len(self.groups), float(max_norm), self.norm, self.coef)
        return self.norm, self.coef

    def step(self, lr: float, eps: float, clip_norm: float | None = None) -> None:
        """Forward, sort and update of the bound batch (one micro-batch):
        without a clip the sort and the update are one fused op,
        ``mdl_hip::fused_backward_rowwise_adagrad_``."""

        if self.k > 1:
            raise ValueError("a step of several micro-batches is forward(micro_batch=m) for each m, then "
                             "sort() and apply()")
        self.forward()
        if clip_norm is None:
            for g, gs in enumerate(self.groups):
                count, at = self._count(g)
                torch.ops.mdl_hip.fused_backward_rowwise_adagrad_(
                    self._weights, self._states, gs.feats_bwd_dev, len(gs.feats_bwd), gs.tables_dev, len(gs.tables),
                    gs.keys, gs.payload, self._n(), count, at, self.bag_count, None, gs.ws, self.plan.max_dim,
                    self.plan.key_bits, gs.bwd_classes, float(lr), float(eps),
                )
        else:
            self.sort()
            _, coef = self.clip(clip_norm)
            self.apply(lr, eps, coef)

    def capture(self, lr: float, eps: float, clip_norm: float | None = None) -> None:
        """Record step(lr, eps, clip_norm) as one HIP graph; replay() then
        issues every launch of the step at once (the host no longer paces
        short steps).  Nothing runs while recording; the graph reads the
        buffers bound at capture time, so a new batch is copied into them
        before a replay (its lengths may differ).  Call it after one eager
        step, which loads the kernels."""

        self._graph = _capture(self.device, lambda: self.step(lr, eps, clip_norm))

    def replay(self) -> None:
        self._graph.replay()


class _SeqGroup:
    """Device state of one key group of a sequence step: the packed sort
    entries of its features (one scan over their rows places them), its
    tables, backward descriptors and workspace."""

    lo: int
    hi: int
    r0: int
    r1: int
    cap: int
    offsets: Tensor
    scan_ws: Tensor
    keys: Tensor
    payload: Tensor
    feats_bwd: np.ndarray
    feats_bwd_dev: Tensor
    tables: np.ndarray
    tables_dev: Tensor
    bwd_classes: int
    ws: Tensor


class SequenceStep:
    """Fused step over sequence features (long user-behaviour histories).

    Every feature ``f`` has a table, right-padded ids ``[B, L_in]``, lengths
    ``[B]`` and a padded output window ``[B, L_out, dim]`` (+ mask); the
    backward reads the window's gradient.  Forward: one gather launch per
    feature; backward: one sort and one segment-reduce + row-wise Adagrad over
    all features together.

    Sort keys are packed: row b of feature f keeps min(len, L_out) entries
    (its window positions; none for an empty input, and a length past the
    input repeats its last id as the reference's window does), placed each
    step by one scan of those clamped lengths on the device, so the backward
    sorts no padding and any lengths of a later batch are honoured.

    A plan of 2^32 - 1 rows or more is cut into key groups
    (``GroupPlan.groups``): each group's features pack their entries into a
    key buffer of their own, placed by a scan over their rows only, and each
    group has its own sort and reduce.

    ``micro_batches=k`` accumulates gradients as ``SparseStep`` does: k
    lists of outputs, masks and gradients; ``forward(micro_batch=m)`` for each
    bound micro-batch, then one ``sort()`` + ``apply()`` update every row once
    with the sum of the k micro-batches' gradients (src/train.py:5388-5396).
    """

    def __init__(
        self,
        plan: ops.GroupPlan,
        ids: Sequence[Tensor],
        lengths: Sequence[Tensor],
        outputs: Sequence[Tensor],
        masks: Sequence[Tensor],
        grads: Sequence[Tensor],
        *,
        order: str = "oldest_to_newest",
        error_count: Tensor | None = None,
        micro_batches: int = 1,
    ) -> None:
        for t in plan.tables:
            if t.state is None:
                raise RuntimeError("every table needs a row-wise Adagrad accumulator")
        self.k = int(micro_batches)
        if self.k < 1:
            raise ValueError("micro_batches must be positive")
        self._looked_up: set[int] = set()  # micro-batches forwarded since the last sort
        if self.k == 1:
            outputs, masks, grads = [outputs], [masks], [grads]
        elif not len(outputs) == len(masks) == len(grads) == self.k:
            raise ValueError("one list of outputs, masks and gradients per micro-batch")
        self.plan = plan
        groups = plan.groups  # row bases of the tables within their key group
        self.device = ids[0].device
        self.ids = [_as_ids(t) for t in ids]
        self.lengths = [t.to(torch.int64).contiguous() for t in lengths]
        self.all_outputs = [list(o) for o in outputs]
        self.all_masks = [list(m) for m in masks]
        self.all_grads = [[g.contiguous() for g in gs] for gs in grads]
        self.outputs, self.masks, self.grads = self.all_outputs[0], self.all_masks[0], self.all_grads[0]
        if order not in ("oldest_to_newest", "newest_to_oldest"):
            raise ValueError("order must be oldest_to_newest or newest_to_oldest")
        self.order = ops._lib.MDL_SEQ_OLDEST_TO_NEWEST if order == "oldest_to_newest" else ops._lib.MDL_SEQ_NEWEST_TO_OLDEST
        self.error_count = (
            error_count if error_count is not None else torch.zeros(1, dtype=torch.int32, device=self.device)
        )
        self.batch = [int(t.size(0)) for t in self.ids]
        # Sort entries a row can hold: its window entries, at most the
        # window's width (none for an empty input).
        self.caps = [int(o.size(1)) if int(i.size(1)) > 0 else 0 for i, o in zip(self.ids, self.outputs)]
        for m in range(1, self.k):
            if [tuple(o.shape) for o in self.all_outputs[m]] != [tuple(o.shape) for o in self.outputs]:
                raise ValueError("every micro-batch's windows need the shapes of the first's")
        self.row_base = np.concatenate([[0], np.cumsum(self.batch)]).astype(np.int64)
        total_rows = int(self.row_base[-1])
        # Entries a step can hold: every row at its cap.
        self.capacity = int(sum(b * c for b, c in zip(self.batch, self.caps)))
        self.key_len = torch.empty(max(total_rows, 1), dtype=torch.int64, device=self.device)
        # Window positions of one micro-batch; micro-batch m's payloads (and
        # gradient rows) follow micro-batch m - 1's.
        positions = int(sum(int(o.size(0)) * int(o.size(1)) for o in self.outputs))
        if positions * self.k >= 1 << 32:
            raise ValueError("the micro-batches' window positions exceed the 32-bit gradient-row payload")
        self.fwd_feats = []  # [m][f]
        for m in range(self.k):
            per = []
            payload_base = m * positions
            for f, spec in enumerate(plan.features):
                table = plan.tables[spec.table]
                out = self.all_outputs[m][f]
                B, L_out, _ = out.shape
                rec = ops.sequence_feature(
                    table.weight, state=table.state, padding_idx=spec.padding_idx, out_dtype=spec.out_dtype,
                    row_base=table.row_base, payload_base=payload_base, grad=self.all_grads[m][f],
                )
                rec["table"] = spec.table
                per.append(rec)
                payload_base += int(B) * int(L_out)
            self.fwd_feats.append(per)
        if self.k > 1:
            self._positions = torch.arange(max(self.capacity, 1), dtype=torch.int64, device=self.device)
            sentinel = int(plan.sentinel)
            self._sentinel = sentinel - (1 << 32) if sentinel >= (1 << 31) else sentinel
        self.groups: list[_SeqGroup] = []
        for g in groups:
            gs = _SeqGroup()
            gs.lo, gs.hi = g.lo, g.hi
            gs.r0, gs.r1 = int(self.row_base[g.lo]), int(self.row_base[g.hi])
            gs.cap = int(sum(self.batch[f] * self.caps[f] for f in range(g.lo, g.hi)))
            cap = max(gs.cap, 1)
            gs.offsets = torch.empty(gs.r1 - gs.r0 + 1, dtype=torch.int64, device=self.device)
            gs.scan_ws = ops._workspace(lib().mdl_offsets_workspace_bytes(gs.r1 - gs.r0), self.device)
            gs.keys = torch.empty(cap * self.k, dtype=torch.int32, device=self.device)
            gs.payload = torch.empty(cap * self.k, dtype=torch.int32, device=self.device)
            # the group's features of every micro-batch, micro-batch 0 first
            # (payload bases ascending, as the reduce's feature search needs)
            gs.feats_bwd = np.concatenate([self.fwd_feats[m][f] for m in range(self.k) for f in range(g.lo, g.hi)])
            gs.tables = ops._tables_array(g.plan, gs.feats_bwd[: g.hi - g.lo]).copy()
            if self.k > 1:
                # a table read by k copies of its feature: the reduce finds each
                # payload's feature by search
                gs.tables["feature"] = -1
            gs.bwd_classes = ops.table_classes(gs.tables)
            gs.feats_bwd_dev = ops.upload(gs.feats_bwd, self.device)
            gs.tables_dev = ops.upload(gs.tables, self.device)
            gs.ws = ops._workspace(
                lib().mdl_backward_workspace_bytes(self._n(gs), len(gs.tables), plan.max_dim), self.device
            )
            self.groups.append(gs)
        # what the update mutates, named in the ops' schemas
        self._weights = [t.weight for t in plan.tables]
        self._states = [t.state for t in plan.tables]

    def _n(self, gs: _SeqGroup) -> int:
        return max(gs.cap, 1) * self.k if self.k > 1 else gs.cap

    def bind(self, ids: Sequence[Tensor] | None = None, lengths: Sequence[Tensor] | None = None) -> None:
        """Point the next steps at another batch (same shapes; any lengths)."""

        if ids is not None:
            new = [_as_ids(t) for t in ids]
            if [tuple(t.shape) for t in new] != [tuple(t.shape) for t in self.ids]:
                raise ValueError("sequence ids must keep their [B, L_in] shapes")
            self.ids = new
        if lengths is not None:
            new = [t.to(torch.int64).contiguous() for t in lengths]
            if [tuple(t.shape) for t in new] != [tuple(t.shape) for t in self.lengths]:
                raise ValueError("sequence lengths must keep their [B] shapes")
            self.lengths = new

    @property
    def count(self) -> Tensor:
        """Device int64 [1]: packed sort entries of the bound batch."""

        if len(self.groups) == 1:
            return self.groups[0].offsets[-1:]
        return torch.stack([gs.offsets[-1] for gs in self.groups]).sum().reshape(1)

    def _stream(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    def forward(self, micro_batch: int = 0) -> None:
        """Window gather (+ packed sort keys) of the bound batch, as
        micro-batch ``micro_batch`` of an accumulated step."""

        mb = int(micro_batch)
        if not 0 <= mb < self.k:
            raise ValueError(f"micro_batch must be in [0, {self.k})")
        self._looked_up.add(mb)
        s = self._stream()
        # Entries each row keeps (its positions that reach the window), then
        # one scan over each key group's rows places them.
        for f, ln in enumerate(self.lengths):
            b0, b1 = int(self.row_base[f]), int(self.row_base[f + 1])
            torch.clamp(ln, 0, self.caps[f], out=self.key_len[b0:b1])
        for gs in self.groups:
            nrows = gs.r1 - gs.r0
            check(
                lib().mdl_lengths_to_offsets(self.key_len.data_ptr() + 8 * gs.r0, nrows, gs.offsets.data_ptr(),
                                             gs.scan_ws.data_ptr(), gs.scan_ws.numel(), s),
                "mdl_lengths_to_offsets",
            )
            region = mb * max(gs.cap, 1)
            for f in range(gs.lo, gs.hi):
                rec = self.fwd_feats[mb][f]
                ids = self.ids[f]
                out = self.all_outputs[mb][f]
                check(
                    lib().mdl_sequence_forward(
                        rec.ctypes.data, ids.data_ptr(), self.lengths[f].data_ptr(), ids.size(0), ids.size(1),
                        out.size(1), self.order, out.data_ptr(), self.all_masks[mb][f].data_ptr(),
                        gs.keys.data_ptr() + 4 * region, gs.payload.data_ptr() + 4 * region,
                        gs.offsets.data_ptr() + 8 * (int(self.row_base[f]) - gs.r0), self.plan.sentinel,
                        self.error_count.data_ptr(), s,
                    ),
                    "mdl_sequence_forward",
                )
            if self.k > 1:
                # entries of the region past this micro-batch's keys sort last
                # and reduce nowhere
                cap = max(gs.cap, 1)
                live = gs.offsets[nrows]
                gs.keys[region: region + cap].masked_fill_(self._positions[:cap] >= live, self._sentinel)

    _check_micro_batches = SparseStep._check_micro_batches

    def sort(self) -> None:
        self._check_micro_batches()
        for gs in self.groups:
            torch.ops.mdl_hip.backward_sort_(
                gs.tables_dev, len(gs.tables), gs.keys, gs.payload, self._n(gs),
                gs.offsets if self.k == 1 else None, gs.r1 - gs.r0, self.plan.max_dim, self.plan.key_bits, gs.ws,
            )

    def apply(self, lr: float, eps: float) -> None:
        for gs in self.groups:
            torch.ops.mdl_hip.backward_apply_(
                self._weights, self._states, gs.feats_bwd_dev, len(gs.feats_bwd), gs.tables_dev, len(gs.tables),
                gs.keys, gs.payload, self._n(gs), None, None, gs.ws, self.plan.max_dim, self.plan.key_bits,
                gs.bwd_classes, float(lr), float(eps),
            )

    def capture(self, lr: float, eps: float) -> None:
        """One HIP graph of step(lr, eps); see SparseStep.capture."""

        self._graph = _capture(self.device, lambda: self.step(lr, eps))

    def replay(self) -> None:
        self._graph.replay()

    def step(self, lr: float, eps: float) -> None:
        """Forward, sort and update of the bound batch (one micro-batch)."""

        if self.k > 1:
            raise ValueError("a step of several micro-batches is forward(micro_batch=m) for each m, then "
                             "sort() and apply()")
        self.forward()
        self.sort()
        self.apply(lr, eps)
