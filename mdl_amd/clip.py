"""Sparse gradient clipping of the trainer, on HIP kernels.

Drop-ins for ``_gradient_values``, ``_gradient_squared_norm``,
``_scale_gradients`` and ``_clip_sparse_grad_norm`` (src/train.py:5730-5826):
the global 2-norm of every sparse (coalesced values) and dense gradient is
one multi-tensor sum of squares, the coefficient
``min(max_norm / (norm + 1e-6), 1)`` is computed on the device, and one
multi-tensor kernel scales every gradient in place in its own dtype -- no host
synchronisation, like the reference's on-device clamp.  The fused training
step (``SparseStep.step(..., clip_norm=...)``) clips inside the backward
instead, without materialising the coalesced gradient.

Only one GPU is supported: with ``torch.distributed`` initialised over more
than one rank, sharded parameters raise (the reference all-reduces their
squared norm, src/train.py:5812-5817).
"""

from __future__ import annotations

import torch
import torch.distributed as torch_dist
from torch import Tensor, nn

from . import ops
from .optim import coalesced_grad


@torch.no_grad()
def _gradient_values(parameters: list[nn.Parameter]) -> list[Tensor]:
    """Coalesced values of sparse grads (stored back) and dense grads as is."""

    grads: list[Tensor] = []
    for parameter in parameters:
        if parameter.grad is None:
            continue
        if parameter.grad.is_sparse:
            grads.append(coalesced_grad(parameter)._values())
        else:
            grads.append(parameter.grad)
    return grads


def _gradient_squared_norm(grads: list[Tensor], device: torch.device) -> Tensor:
    """Sum of the squared fp32 2-norms of ``grads``: a 0-d fp32 tensor."""

    return ops.grad_sumsq([g.detach() for g in grads], device).reshape(())


def _scale_gradients(grads: list[Tensor], coefficient: Tensor) -> None:
    """``grad *= coefficient`` in place, the coefficient cast to each grad's dtype."""

    if not grads:
        return
    coef = coefficient.detach().reshape(1).to(device=grads[0].device, dtype=torch.float32)
    ops.scale_(grads, coef)


@torch.no_grad()
def _clip_sparse_grad_norm(
    replicated_parameters: list[nn.Parameter],
    sharded_parameters: list[nn.Parameter],
    max_norm: float,
) -> Tensor:
    """Clip one logical sparse group to ``max_norm``; returns the pre-clip norm.

    One ``mdl_hip::clip_sparse_grad_norm_`` call: the C++ extension takes
    every parameter's gradient values (coalescing and storing back a sparse
    gradient that is neither coalesced nor the lookup's capacity-sized one),
    sums their squares per list, forms min(max_norm / (norm + 1e-6), 1) and
    scales every gradient in place, all on the device."""

    if (
        sharded_parameters
        and torch_dist.is_available()
        and torch_dist.is_initialized()
        and torch_dist.get_world_size() > 1
    ):
        raise NotImplementedError("sparse clipping across ranks is outside this single-GPU build")
    params = [p for p in [*replicated_parameters, *sharded_parameters] if p.device is not None]
    if not params:
        return torch.tensor(0.0)
    return torch.ops.mdl_hip.clip_sparse_grad_norm_(list(replicated_parameters), list(sharded_parameters),
                                                    float(max_norm))
