"""One fused sparse step over fixed device buffers.

``SparseStep`` binds a feature layout (:class:`mdl_amd.ops.GroupPlan`) to
persistent buffers -- packed ids, concatenated bag lengths, pooled outputs,
upstream gradients -- and builds every descriptor, chunk table and workspace
once.  A step is then launches only, with no host work, allocation or sync:

    lengths -> offsets scan, grouped lookup + pooling (+ sort keys),
    radix sort, segment reduction + row-wise Adagrad.

This is the path of a training loop whose batch layout is fixed (same
features, batch size and bag-count per feature), e.g. with the pooled outputs
written straight into the RankMixer token-slot buffer ``[B, sum(dim)]``.
"""

from __future__ import annotations

from typing import Sequence

import numpy as np
import torch
from torch import Tensor

from . import ops
from ._lib import CHUNK_DTYPE, MDL_POOL_NONE, check, lib


def _capture(device: torch.device, fn) -> "torch.cuda.CUDAGraph":
    """fn's launches recorded on a side stream of default priority."""

    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(device=device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.graph(graph, stream=side):
        fn()
    torch.cuda.current_stream(device).wait_stream(side)
    return graph


class SparseStep:
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
    ) -> None:
        for t in plan.tables:
            if t.state is None:
                raise RuntimeError("every table needs a row-wise Adagrad accumulator")
        self.plan = plan
        self.device = packed_ids.device
        self.ids = packed_ids.contiguous()
        self.n = int(self.ids.numel())
        pooled_any = any(s.pooling != MDL_POOL_NONE for s in plan.features)
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
        out_ptrs = [o.data_ptr() for o in outputs]
        out_strides = [o.stride(0) if o.ndim == 2 else int(o.size(-1)) for o in outputs]
        self.feats_fwd = ops.build_features(plan, id_counts, bag_counts, out_ptrs, out_strides)
        target = ops.forward_target_ids(self.feats_fwd)
        n_chunks = lib().mdl_plan_chunks(self.feats_fwd.ctypes.data, len(self.feats_fwd), target, None, 0)
        if n_chunks < 0:
            check(int(n_chunks), "mdl_plan_chunks")
        chunks = np.zeros(max(n_chunks, 1), dtype=CHUNK_DTYPE)
        lib().mdl_plan_chunks(self.feats_fwd.ctypes.data, len(self.feats_fwd), target, chunks.ctypes.data,
                              n_chunks)
        self.n_chunks = int(n_chunks)
        res = ops.ForwardResult(
            plan=plan, device=self.device, ids=self.ids, offsets=None, outputs=list(outputs),
            feats=self.feats_fwd, keys=None, payload=None, bag_count=None, error_count=self.error_count,
        )
        self.feats_bwd, self._grads = ops._attach_grads(res, grads)
        self.tables = ops._tables_array(plan, self.feats_bwd)
        self.fwd_classes = ops.feature_classes(self.feats_fwd)
        self.bwd_classes = ops.table_classes(self.tables)
        self.feats_fwd_dev = ops.upload(self.feats_fwd, self.device)
        self.chunks_dev = ops.upload(chunks, self.device)
        self.feats_bwd_dev = ops.upload(self.feats_bwd, self.device)
        self.tables_dev = ops.upload(self.tables, self.device)
        total_rows = int(
            np.where(self.feats_fwd["pooling"] != MDL_POOL_NONE, self.feats_fwd["num_bags"],
                     self.feats_fwd["num_ids"]).sum()
        )
        self.keys = torch.empty(max(self.n, 1), dtype=torch.int32, device=self.device)
        self.payload = torch.empty(max(self.n, 1), dtype=torch.int32, device=self.device)
        self.bag_count = (
            torch.empty(max(total_rows, 1), dtype=torch.float32, device=self.device) if pooled_any else None
        )
        self.ws = ops._workspace(
            lib().mdl_backward_workspace_bytes(self.n, len(self.tables), plan.max_dim), self.device
        )
        self.sumsq = torch.zeros(1, dtype=torch.float32, device=self.device)
        self.norm = torch.zeros(1, dtype=torch.float32, device=self.device)
        self.coef = torch.ones(1, dtype=torch.float32, device=self.device)

    def _stream(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    def forward(self) -> None:
        """Offsets scan + grouped lookup/pooling (+ backward sort keys)."""

        s = self._stream()
        if self.offsets is not None:
            check(
                lib().mdl_lengths_to_offsets(
                    self.lengths.data_ptr(), self.lengths.numel(), self.offsets.data_ptr(),
                    self.scan_ws.data_ptr(), self.scan_ws.numel(), s,
                ),
                "mdl_lengths_to_offsets",
            )
        check(
            lib().mdl_forward(
                self.feats_fwd_dev.data_ptr(), len(self.feats_fwd), self.chunks_dev.data_ptr(), self.n_chunks,
                self.ids.data_ptr(), ops._ptr(self.offsets), self.keys.data_ptr(), self.payload.data_ptr(),
                self.plan.sentinel, ops._ptr(self.bag_count), self.error_count.data_ptr(), self.fwd_classes, s,
            ),
            "mdl_forward",
        )

    def sort(self) -> None:
        """Radix sort of the (row, gradient-row) pairs + chunk plan."""

        check(
            lib().mdl_backward_sort(
                self.tables_dev.data_ptr(), len(self.tables), self.plan.max_dim, self.keys.data_ptr(),
                self.payload.data_ptr(), self.n, self.plan.key_bits, self.ws.data_ptr(), self.ws.numel(),
                self._stream(),
            ),
            "mdl_backward_sort",
        )

    def _bwd_args(self) -> tuple:
        return (
            self.feats_bwd_dev.data_ptr(), len(self.feats_bwd), self.tables_dev.data_ptr(), len(self.tables),
            self.plan.max_dim, self.keys.data_ptr(), self.payload.data_ptr(), self.n, self.plan.key_bits,
            ops._ptr(self.bag_count),
        )

    def apply(self, lr: float, eps: float, grad_scale: Tensor | None = None) -> None:
        """Segment reduction of duplicate rows + fused row-wise Adagrad
        (gradients times ``grad_scale``, a device fp32 [1], when given)."""

        check(
            lib().mdl_backward_apply(
                *self._bwd_args(), float(lr), float(eps), ops._ptr(grad_scale), self.ws.data_ptr(),
                self.ws.numel(), self.bwd_classes, self._stream(),
            ),
            "mdl_backward_apply",
        )

    def clip(self, max_norm: float) -> tuple[Tensor, Tensor]:
        """After sort(): (pre-clip global norm, clip coefficient), on device.

        The norm is that of the coalesced gradient of every table, as the
        trainer's sparse clip computes it (src/train.py:5788-5826)."""

        check(
            lib().mdl_backward_sumsq(
                *self._bwd_args(), self.sumsq.data_ptr(), self.ws.data_ptr(), self.ws.numel(), self.bwd_classes,
                self._stream(),
            ),
            "mdl_backward_sumsq",
        )
        check(
            lib().mdl_clip_coef(self.sumsq.data_ptr(), 1, float(max_norm), self.norm.data_ptr(),
                                self.coef.data_ptr(), self._stream()),
            "mdl_clip_coef",
        )
        return self.norm, self.coef

    def step(self, lr: float, eps: float, clip_norm: float | None = None) -> None:
        self.forward()
        self.sort()
        if clip_norm is None:
            self.apply(lr, eps)
        else:
            _, coef = self.clip(clip_norm)
            self.apply(lr, eps, coef)

    def capture(self, lr: float, eps: float, clip_norm: float | None = None) -> None:
        """Record step(lr, eps, clip_norm) as one HIP graph; replay() then
        issues every launch of the step at once (the host no longer paces
        short steps).  Nothing runs while recording; the step's buffers are
        its own, so a new batch of the same layout is copied into them before
        a replay.  Call it after one eager step, which loads the kernels."""

        self._graph = _capture(self.device, lambda: self.step(lr, eps, clip_norm))

    def replay(self) -> None:
        self._graph.replay()


class SequenceStep:
    """Fused step over sequence features (long user-behaviour histories).

    Every feature ``f`` has a table, right-padded ids ``[B, L_in]``, lengths
    ``[B]`` and a padded output window ``[B, L_out, dim]`` (+ mask); the
    backward reads the window's gradient.  Forward: one gather launch per
    feature; backward: one sort and one segment-reduce + row-wise Adagrad over
    all features together.
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
    ) -> None:
        for t in plan.tables:
            if t.state is None:
                raise RuntimeError("every table needs a row-wise Adagrad accumulator")
        self.plan = plan
        self.device = ids[0].device
        self.ids = [t.contiguous() for t in ids]
        self.lengths = [t.to(torch.int64).contiguous() for t in lengths]
        self.outputs = list(outputs)
        self.masks = list(masks)
        self.grads = [g.contiguous() for g in grads]
        self.order = ops._lib.MDL_SEQ_OLDEST_TO_NEWEST if order == "oldest_to_newest" else ops._lib.MDL_SEQ_NEWEST_TO_OLDEST
        self.error_count = (
            error_count if error_count is not None else torch.zeros(1, dtype=torch.int32, device=self.device)
        )
        # Sort keys are packed: row b of feature f keeps min(len, L_in, L_out)
        # entries (the positions that reach the window), so the backward
        # sorts no padding.  The lengths are read once here, like the id
        # counts of SparseStep: a step object serves one batch layout.
        feats = []
        self.fwd_feats = []
        key_off = 0
        payload_base = 0
        self.key_offsets = []
        self.row_offsets = []
        for f, spec in enumerate(plan.features):
            out = self.outputs[f]
            L_in = int(self.ids[f].size(1))
            kept = np.clip(self.lengths[f].cpu().numpy(), 0, min(L_in, int(out.size(1))))
            offs = np.zeros(kept.size + 1, dtype=np.int64)
            np.cumsum(kept, out=offs[1:])
            self.row_offsets.append(ops.upload(offs, self.device))
            self.key_offsets.append(key_off)
            key_off += int(offs[-1])
        self.n = key_off
        self.keys = torch.empty(max(self.n, 1), dtype=torch.int32, device=self.device)
        self.payload = torch.empty(max(self.n, 1), dtype=torch.int32, device=self.device)
        for f, spec in enumerate(plan.features):
            table = plan.tables[spec.table]
            out = self.outputs[f]
            B, L_out, _ = out.shape
            rec = ops.sequence_feature(
                table.weight, state=table.state, padding_idx=spec.padding_idx, out_dtype=spec.out_dtype,
                row_base=table.row_base, payload_base=payload_base, grad=self.grads[f],
            )
            rec["table"] = spec.table
            feats.append(rec)
            self.fwd_feats.append(rec.copy())
            payload_base += int(B) * int(L_out)
        self.feats_bwd = np.concatenate(feats)
        self.tables = ops._tables_array(plan, self.feats_bwd)
        self.bwd_classes = ops.table_classes(self.tables)
        self.feats_bwd_dev = ops.upload(self.feats_bwd, self.device)
        self.tables_dev = ops.upload(self.tables, self.device)
        self.ws = ops._workspace(
            lib().mdl_backward_workspace_bytes(self.n, len(self.tables), plan.max_dim), self.device
        )

    def _stream(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    def forward(self) -> None:
        s = self._stream()
        for f, rec in enumerate(self.fwd_feats):
            ids = self.ids[f]
            out = self.outputs[f]
            off = self.key_offsets[f]
            check(
                lib().mdl_sequence_forward(
                    rec.ctypes.data, ids.data_ptr(), self.lengths[f].data_ptr(), ids.size(0), ids.size(1),
                    out.size(1), self.order, out.data_ptr(), self.masks[f].data_ptr(),
                    self.keys.data_ptr() + 4 * off, self.payload.data_ptr() + 4 * off,
                    self.row_offsets[f].data_ptr(), self.plan.sentinel, self.error_count.data_ptr(), s,
                ),
                "mdl_sequence_forward",
            )

    def sort(self) -> None:
        check(
            lib().mdl_backward_sort(
                self.tables_dev.data_ptr(), len(self.tables), self.plan.max_dim, self.keys.data_ptr(),
                self.payload.data_ptr(), self.n, self.plan.key_bits, self.ws.data_ptr(), self.ws.numel(),
                self._stream(),
            ),
            "mdl_backward_sort",
        )

    def apply(self, lr: float, eps: float) -> None:
        check(
            lib().mdl_backward_apply(
                self.feats_bwd_dev.data_ptr(), len(self.feats_bwd), self.tables_dev.data_ptr(), len(self.tables),
                self.plan.max_dim, self.keys.data_ptr(), self.payload.data_ptr(), self.n, self.plan.key_bits,
                None, float(lr), float(eps), None, self.ws.data_ptr(), self.ws.numel(), self.bwd_classes,
                self._stream(),
            ),
            "mdl_backward_apply",
        )

    def capture(self, lr: float, eps: float) -> None:
        """One HIP graph of step(lr, eps); see SparseStep.capture."""

        self._graph = _capture(self.device, lambda: self.step(lr, eps))

    def replay(self) -> None:
        self._graph.replay()

    def step(self, lr: float, eps: float) -> None:
        self.forward()
        self.sort()
        self.apply(lr, eps)
