"""Bag pooling of already-embedded rows, on the HIP pooling kernel.

Drop-ins for the model's pooling helpers:

* ``_mean_pool_categorical_bag(embedded, indices, lengths, null_policy)``
  (src/model.py:509-587): flat ``[N, D]/[N]/[B]`` or padded
  ``[B, L, D]/[B, L]/[B]`` inputs, ``"exclude"`` / ``"include_as_padding"``
  null policies, ``sums / max(counts, 1)``, empty bags pool to 0.
* ``_batch_mean_pool_flat_bags(bags)`` (src/model.py:590-678): every flat bag
  of the call is pooled in ONE launch, whatever its dtype, dim or policy
  (the reference groups by ``(dtype, dim, policy, batch)`` and launches once
  per group); padded bags go through the single-bag path.

The forward is ``mdl_forward`` over features flagged
``MDL_FLAG_ROWS_BY_POSITION`` (row i of ``embedded`` is id slot i; the ids
only decide null weights); the backward is ``mdl_pool_backward``, which
writes ``grad[bag] * w_i / max(count, 1)`` into every position row, the
autograd of the reference's ``index_add_`` + division (src/model.py:564-570).
Sums are taken in fp32 and rounded once to the embedded dtype (the reference
accumulates in the embedded dtype, so bf16 results agree within bf16
rounding).  Inputs must be float32 or bfloat16 tensors on the ROCm device.
"""

from __future__ import annotations

from typing import Sequence

import numpy as np
import torch
from torch import Tensor

from . import ops
from .embeddings import _deferred_counter, deferred_index_checks

_POLICIES = ("exclude", "include_as_padding")


def _check_flat(embedded: Tensor, indices: Tensor, lengths: Tensor) -> None:
    if embedded.size(0) != indices.size(0):
        raise ValueError("categorical bag flat values and embeddings are misaligned")
    if lengths.numel() == 0 and indices.numel() != 0:
        raise ValueError("categorical bag flat length must be zero when lengths is empty")


def _as_flat(
    embedded: Tensor, indices: Tensor, lengths: Tensor, null_policy: str
) -> tuple[Tensor, Tensor, Tensor, str, tuple[int, ...] | None]:
    """(embedded [N, D], ids [N], lengths [B], policy, padded shape or None)."""

    if lengths.ndim != 1:
        raise ValueError("categorical bag lengths must have shape [B]")
    if null_policy not in _POLICIES:
        raise ValueError(f"unsupported categorical bag null policy {null_policy!r}")
    if embedded.ndim == 2 and indices.ndim == 1:
        _check_flat(embedded, indices, lengths)
        return embedded, indices, lengths, null_policy, None
    if embedded.ndim != 3 or indices.ndim != 2:
        raise ValueError(
            "categorical bag tensors must be flat [N,D]/[N]/[B] "
            "or padded [B,L,D]/[B,L]/[B]"
        )
    if embedded.shape[:2] != indices.shape or embedded.size(0) != lengths.numel():
        raise ValueError("categorical bag values, embeddings, and lengths are misaligned")
    # Padded layout: bag b is the L slots of row b; the slots past len_b (and
    # nulls under "exclude") get weight 0, which the kernel's "exclude" rule
    # gives to ids equal to 0, so the ids become the validity mask.
    B, L, D = embedded.shape
    positions = torch.arange(L, device=indices.device).view(1, -1)
    valid = positions < lengths.to(indices.device).view(-1, 1)
    if null_policy == "exclude":
        valid = valid & indices.ne(0)
    flat_lengths = torch.full((B,), L, dtype=torch.int64, device=indices.device)
    return embedded.reshape(B * L, D), valid.reshape(-1).to(torch.int64), flat_lengths, "exclude", tuple(embedded.shape)


class _BagPoolFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, ctl: dict, *embedded: Tensor):  # type: ignore[override]
        plan: ops.GroupPlan = ctl["plan"]
        res = ops.grouped_forward(
            plan, ctl["ids"], ctl["lengths"], with_backward=False, with_bag_count=True,
            error_count=ctl["error_count"],
        )
        _check_lengths(res, ctl)
        ctx.res = res
        ctx.rows = [int(e.size(0)) for e in embedded]
        return tuple(res.outputs)

    @staticmethod
    def backward(ctx, *grads: Tensor):  # type: ignore[override]
        res: ops.ForwardResult = ctx.res
        dests: list[Tensor | None] = []
        for f, spec in enumerate(res.plan.features):
            if not ctx.needs_input_grad[1 + f]:
                dests.append(None)
                continue
            w = res.plan.tables[spec.table].weight
            dests.append(torch.empty((ctx.rows[f], int(w.size(1))), dtype=w.dtype, device=w.device))
        ops.pool_backward(res, list(grads), dests)
        ctx.res = None
        return (None, *dests)


def _check_lengths(res: ops.ForwardResult, ctl: dict) -> None:
    """sum(lengths) must equal the flat length of every bag (src/model.py:529-551)."""

    feats = res.feats
    if len(feats) == 0:
        return
    host = np.stack([feats["bag_base"], feats["bag_base"] + feats["num_bags"], feats["num_ids"]]).astype(np.int64)
    starts, ends, counts = ops.upload(host, res.device).view(torch.int64).view(3, -1)
    mismatched = (res.offsets[ends] - res.offsets[starts]).ne(counts).sum(dtype=torch.int32)
    if ctl["deferred"]:
        res.error_count.add_(mismatched)
        return
    bad = torch.stack([mismatched, res.error_count.reshape(())]).tolist()
    if bad[0]:
        sums = (res.offsets[ends] - res.offsets[starts]).tolist()
        for n, total in zip(feats["num_ids"].tolist(), sums):
            if n != total:
                raise ValueError(f"categorical bag flat length {n} != sum(lengths) {total}")
    if bad[1]:
        raise ValueError("categorical bag lengths must be non-negative")


def pool_bags(
    items: Sequence[tuple[Tensor, Tensor, Tensor, str]], *, mode: str = "mean"
) -> list[Tensor]:
    """Pool every ``(embedded, indices, lengths, null_policy)`` bag in one launch.

    ``mode`` is ``"mean"`` (the reference's only pooling) or ``"sum"``.
    Returns one ``[B, D]`` tensor per item, in the embedded dtype.
    """

    if mode not in ("mean", "sum"):
        raise ValueError(f"unsupported pooling {mode!r}")
    outputs: list[Tensor | None] = [None] * len(items)
    plan = ops.GroupPlan()
    ids: list[Tensor] = []
    lengths: list[Tensor] = []
    inputs: list[Tensor] = []
    slots: list[tuple[int, tuple[int, ...] | None]] = []
    for k, (embedded, indices, lens, policy) in enumerate(items):
        emb, idx, ln, pol, padded = _as_flat(embedded, indices, lens, policy)
        if ln.numel() == 0:
            outputs[k] = embedded.new_zeros((0, embedded.size(-1)))
            continue
        if idx.dtype != torch.long:
            idx = idx.long()
        emb = ops._row_major_aligned(emb)
        plan.add_feature(emb, pooling=mode, null_policy=pol, padding_idx=0, rows_by_position=True)
        ids.append(idx.contiguous())
        lengths.append(ln)
        inputs.append(emb)
        slots.append((k, padded))
    if inputs:
        deferred = deferred_index_checks()
        ctl = {
            "plan": plan,
            "ids": ids,
            "lengths": lengths,
            "deferred": deferred,
            "error_count": _deferred_counter(inputs[0].device) if deferred else None,
        }
        pooled = _BagPoolFn.apply(ctl, *inputs)
        for (k, _), out in zip(slots, pooled):
            outputs[k] = out
    return [o for o in outputs if o is not None]


def _mean_pool_categorical_bag(
    embedded: Tensor,
    indices: Tensor,
    lengths: Tensor,
    null_policy: str,
) -> Tensor:
    """Mean-pool one categorical bag (src/model.py:509-587)."""

    return pool_bags([(embedded, indices, lengths, null_policy)])[0]


def _batch_mean_pool_flat_bags(
    bags: Sequence[tuple[str, Tensor, Tensor, Tensor, str]],
) -> dict[str, Tensor]:
    """Mean-pool many bags with one launch (src/model.py:590-678).

    Returns ``{name: [B, D]}``; numerics match :func:`_mean_pool_categorical_bag`.
    """

    if not bags:
        return {}
    pooled = pool_bags([(e, i, ln, p) for _, e, i, ln, p in bags])
    return {name: out for (name, *_), out in zip(bags, pooled)}
