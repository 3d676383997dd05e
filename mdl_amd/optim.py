"""Drop-in ``ShardedRowWiseAdagrad`` whose update is a gfx950 HIP kernel.

Same constructor, state layout (``step``: 0-d float64 on CPU, ``sum``: one
fp32 accumulator per row) and ``load_state_dict`` behaviour as
src/optim.py:212-377, so checkpoints move between the two unchanged.
Gradients must be sparse COO.  ``step`` is one ``mdl_hip::rowwise_adagrad_step_``
call per parameter group: the C++ extension checks the gradients, advances
the step counts and updates every parameter of a device with one grouped
launch.  A coalesced gradient is used as it is; a capacity-sized gradient of
the grouped lookup is updated up to its row count, read on the device; any
other gradient is coalesced by the library's sort/segment-reduce first, with
no host read.  Parameters on the CPU take the reference's CPU branch
(src/optim.py:359-376).
"""

from __future__ import annotations

import copy
from collections.abc import Iterable
from typing import Any, Callable

import torch
from torch import Tensor, nn

from . import embeddings, library


def coalesced_grad(parameter: Tensor) -> Tensor:
    """The parameter's sparse gradient with every row's summed value once,
    stored back as ``parameter.grad`` (src/train.py:5730-5742).

    A capacity-sized gradient of the lookup is returned as it is: its entries
    past the row count repeat a row with zero values, which changes no norm
    and no scaling (the clip reads only the values).  Any other uncoalesced
    gradient is coalesced exactly on the device (one host read to size it)."""

    grad = parameter.grad
    if library.capacity_grad(parameter, grad) is not None or grad.is_coalesced():
        return grad
    rows, values = torch.ops.mdl_hip.sparse_coalesce(grad._indices()[0], grad._values(), int(parameter.shape[0]))
    parameter.grad = torch.sparse_coo_tensor(rows.unsqueeze(0), values, tuple(grad.shape), is_coalesced=True)
    return parameter.grad


def fused_rowwise_adagrad_update(
    parameter: Tensor,
    accumulator: Tensor,
    rows: Tensor,
    values: Tensor,
    *,
    lr: float,
    eps: float,
) -> None:
    """Row-wise Adagrad for one table (src/optim.py:68-108).

    ``rows`` must be unique.  ``values`` may be bf16 or fp32; the accumulator
    stays fp32 and the weight may be bf16 or fp32 (one rounding on store).
    """

    if rows.numel() == 0:
        return
    torch.ops.mdl_hip.rowwise_adagrad_(parameter, accumulator, rows, values, float(lr), float(eps))


class ShardedRowWiseAdagrad(torch.optim.Optimizer):
    """Row-wise Adagrad: one fp32 accumulator per row (mean of squared grads)."""

    def __init__(
        self,
        params: Iterable[nn.Parameter],
        lr: float,
        lr_decay: float = 0.0,
        weight_decay: float = 0.0,
        initial_accumulator_value: float = 0.0,
        eps: float = 1.0e-10,
        *,
        state_dtype: torch.dtype = torch.float32,
    ) -> None:
        if lr <= 0.0:
            raise ValueError("lr must be positive")
        if lr_decay < 0.0:
            raise ValueError("lr_decay must be non-negative")
        if weight_decay != 0.0:
            raise ValueError(
                "ShardedRowWiseAdagrad does not support weight decay for sparse gradients"
            )
        if initial_accumulator_value < 0.0:
            raise ValueError("initial_accumulator_value must be non-negative")
        if eps <= 0.0:
            raise ValueError("eps must be positive")
        defaults = {
            "lr": lr,
            "lr_decay": lr_decay,
            "weight_decay": weight_decay,
            "initial_accumulator_value": initial_accumulator_value,
            "eps": eps,
            "state_dtype": state_dtype,
        }
        super().__init__(params, defaults)
        for group in self.param_groups:
            for parameter in group["params"]:
                if parameter.ndim != 2:
                    raise ValueError("ShardedRowWiseAdagrad expects 2D embedding parameters")
                state = self.state[parameter]
                state["step"] = torch.zeros((), dtype=torch.float64)
                state["sum"] = torch.full(
                    (parameter.shape[0],),
                    float(initial_accumulator_value),
                    dtype=state_dtype,
                    device=parameter.device,
                )

    def load_state_dict(self, state_dict: dict[str, Any]) -> None:
        # The base class casts state tensors to the parameter dtype; restore
        # the fp32 accumulators and CPU float64 steps from a snapshot.
        original = copy.deepcopy(state_dict)
        super().load_state_dict(state_dict)
        saved_items: list[dict[str, Any]] = []
        for group in original.get("param_groups", ()):
            for param_id in group["params"]:
                saved_items.append(original.get("state", {}).get(param_id, {}))
        index = 0
        for group in self.param_groups:
            state_dtype = group.get("state_dtype", torch.float32)
            for parameter in group["params"]:
                saved = saved_items[index] if index < len(saved_items) else {}
                index += 1
                state = self.state.get(parameter)
                if not state:
                    continue
                accumulator = saved.get("sum", state.get("sum"))
                if isinstance(accumulator, Tensor):
                    state["sum"] = accumulator.to(device=parameter.device, dtype=state_dtype)
                step = saved.get("step", state.get("step"))
                if isinstance(step, Tensor):
                    state["step"] = step.to(device="cpu", dtype=torch.float64)

    def zero_grad(self, set_to_none: bool = True) -> None:
        """``torch.optim.Optimizer.zero_grad``; with ``set_to_none`` (the
        trainer's call, src/train.py:6955,7005) one call of the extension per
        parameter group resets every gradient."""

        if not set_to_none:
            super().zero_grad(set_to_none=False)
            return
        for group in self.param_groups:
            torch.ops.mdl_hip.clear_grads_(group["params"])

    @torch.no_grad()
    def step(self, closure: Callable[[], Tensor] | None = None) -> Tensor | None:
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        if embeddings.deferred_index_checks():
            embeddings.check_index_errors()
        # One call per parameter group: the extension checks every gradient,
        # advances the CPU step counts, decays the learning rates and updates
        # every device parameter with one grouped launch per device (CPU
        # parameters take the reference's CPU branch, src/optim.py:359-376).
        for group in self.param_groups:
            params = group["params"]
            states = [self.state[p] for p in params]
            torch.ops.mdl_hip.rowwise_adagrad_step_(
                params, [st["sum"] for st in states], [st["step"] for st in states], [p.grad for p in params],
                float(group["lr"]), float(group["lr_decay"]), float(group["eps"]),
            )
        return loss
