"""PyTorch CPU restatement of the reference sparse step -- TEST AND BASELINE
INFRASTRUCTURE ONLY.

Like ``oracle.py``, only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` use this module; the product
(``mdl_amd``) never imports it.  It is the reference's single-rank CPU path,
call for call, and it is what the bench times as the CPU baseline:

* lookup: ``F.embedding(ids, W, padding_idx=0, sparse=True)``
  (src/embeddings.py:468-473, single rank :751-779);
* pooling: ``repeat_interleave`` segment ids, ``index_add_`` of the weighted
  rows and of the weights, ``sums / counts.clamp(min=1)``
  (src/model.py:552-570); sum pooling keeps the sums (the reference has mean
  pooling only; sum is its numerator);
* backward: autograd of the linear loss ``sum(out_f * grad_f)``, which hands
  every table a sparse COO gradient;
* coalesce: ``grad.coalesce()`` (src/optim.py:321-324);
* update: the CPU branch of ``ShardedRowWiseAdagrad.step``
  (src/optim.py:359-376) -- ``acc.index_add_(rows, mean(g^2, 1))``,
  ``den = sqrt(acc[rows]) + eps``, ``W.index_add_(rows, g / den, alpha=-lr)``.

Pinned against the C oracle (``oracle.sparse_step``) in
``tests/test_oracle.py``.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import Tensor


@dataclass
class Feature:
    table: int
    pooling: str  # "none" | "sum" | "mean"
    null_policy: str = "exclude"


def pool(embedded: Tensor, ids: Tensor, lengths: Tensor, pooling: str, null_policy: str) -> Tensor:
    """Flat-bag pooling of already-embedded rows (src/model.py:552-570)."""

    batch = int(lengths.numel())
    weights = ids.ne(0).to(embedded.dtype) if null_policy == "exclude" else embedded.new_ones(ids.shape)
    seg = torch.repeat_interleave(torch.arange(batch, dtype=torch.long), lengths.long())
    sums = embedded.new_zeros((batch, embedded.size(-1)))
    counts = embedded.new_zeros((batch,))
    if seg.numel():
        sums.index_add_(0, seg, embedded * weights.unsqueeze(-1))
        counts.index_add_(0, seg, weights)
    if pooling == "sum":
        return sums
    return sums / counts.clamp(min=1).unsqueeze(-1)


def rowwise_adagrad_cpu(weight: Tensor, acc: Tensor, grad: Tensor, lr: float, eps: float) -> None:
    """The CPU branch of ShardedRowWiseAdagrad.step for one parameter."""

    grad = grad.coalesce()
    rows = grad.indices()[0]
    values = grad.values()
    if rows.numel() == 0:
        return
    state_values = values if values.dtype == torch.float32 else values.float()
    acc.index_add_(0, rows, state_values.square().mean(dim=1))
    den = acc.index_select(0, rows).sqrt_().add_(eps).unsqueeze(1)
    update = state_values / den
    if update.dtype != weight.dtype:
        update = update.to(dtype=weight.dtype)
    weight.index_add_(0, rows, update, alpha=-lr)


class TorchStep:
    """Fwd + bwd + row-wise Adagrad of a grouped batch on CPU tensors.

    ``tables``: ``[rows, dim]`` weights (updated in place) and ``accs`` their
    fp32 accumulators; ``features``: which table each feature reads and how it
    pools.  ``step`` takes per-feature ids (and bag lengths for pooled
    features) and upstream gradients of the outputs, and returns the outputs.
    """

    def __init__(self, tables: list[Tensor], accs: list[Tensor], features: list[Feature]) -> None:
        self.params = [torch.nn.Parameter(t, requires_grad=True) for t in tables]
        self.accs = accs
        self.features = features

    def step(self, ids: list[Tensor], lengths: list[Tensor | None], grads: list[Tensor], lr: float,
             eps: float) -> list[Tensor]:
        for p in self.params:
            p.grad = None
        outs = []
        loss = None
        for f, x, ln, g in zip(self.features, ids, lengths, grads):
            emb = F.embedding(x, self.params[f.table], padding_idx=0, sparse=True)
            out = emb if f.pooling == "none" else pool(emb, x, ln, f.pooling, f.null_policy)
            term = (out * g).sum()
            loss = term if loss is None else loss + term
            outs.append(out.detach())
        loss.backward()
        with torch.no_grad():
            for p, acc in zip(self.params, self.accs):
                if p.grad is not None:
                    rowwise_adagrad_cpu(p.data, acc, p.grad, lr, eps)
        return outs
