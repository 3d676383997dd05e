"""Drop-in ``ShardedEmbedding`` and grouped lookup on one MI355X.

Public surface of src/embeddings.py for the single-GPU path
(``world_size == 1``, src/embeddings.py:752-779 and :1675-1709): the module
keeps the reference constructor, attributes, parameter/state layout and
sparse-COO gradient contract, but every lookup is one launch of the gfx950
gather kernel and every backward is the deterministic sort/segment-reduce of
libmdl_hip, which hands autograd an already-coalesced gradient.

Multi-GPU owner routing (all-to-all) is not part of this build: a process
group with more than one rank raises ``NotImplementedError``.
"""

from __future__ import annotations

from contextlib import contextmanager
from dataclasses import asdict, dataclass
from hashlib import sha256
import json
import threading
from typing import Any, Iterable, Iterator, Literal

import torch
import torch.distributed as torch_dist
from torch import Tensor, nn

from . import library, ops  # noqa: F401  (library registers the mdl_hip ops)

_STATS_HOST_SYNC = threading.local()
_DEFERRED = threading.local()

EmbeddingShardStrategy = Literal["row_wise", "table_wise"]
OptimizerStateLayout = Literal["full", "rowwise"]


# ------------------------------------------------------------ stats flags --


def embedding_stats_host_sync_enabled() -> bool:
    return bool(getattr(_STATS_HOST_SYNC, "enabled", True))


def set_embedding_stats_host_sync(enabled: bool) -> None:
    _STATS_HOST_SYNC.enabled = bool(enabled)


@contextmanager
def embedding_stats_host_sync(enabled: bool) -> Iterator[None]:
    previous = getattr(_STATS_HOST_SYNC, "enabled", True)
    _STATS_HOST_SYNC.enabled = bool(enabled)
    try:
        yield
    finally:
        _STATS_HOST_SYNC.enabled = previous


# ------------------------------------------------------------- id checks --
#
# Ids outside [0, num_embeddings) are looked up as zero rows and counted on
# the device.  How the count is checked on a ROCm device:
#   "async" (default): torch._assert_async on the count -- no host sync, a
#       device-side assert on failure, as the reference does on GPU
#       (src/embeddings.py:140-147);
#   "sync": one host read per lookup and the reference's IndexError naming
#       the table and the first ids (the reference's CPU behaviour);
#   "deferred": the count is added to a per-device counter and the next
#       optimizer step (or check_index_errors()) raises IndexError.
# CPU tensors always raise IndexError at once, like the reference's CPU path.
_CHECK_MODES = ("async", "sync", "deferred")


def set_index_check_mode(mode: str) -> None:
    if mode not in _CHECK_MODES:
        raise ValueError(f"index check mode must be one of {_CHECK_MODES}")
    _DEFERRED.mode = mode


def index_check_mode() -> str:
    return getattr(_DEFERRED, "mode", "async")


def set_deferred_index_checks(enabled: bool) -> None:
    """Deferred mode on (True) or back to the default asynchronous assert."""

    set_index_check_mode("deferred" if enabled else "async")


def deferred_index_checks() -> bool:
    return index_check_mode() == "deferred"


_DEFERRED_COUNTERS: dict[torch.device, Tensor] = {}


def _deferred_counter(device: torch.device) -> Tensor:
    t = _DEFERRED_COUNTERS.get(device)
    if t is None:
        t = torch.zeros(1, dtype=torch.int32, device=device)
        _DEFERRED_COUNTERS[device] = t
    return t


def check_index_errors() -> None:
    """Raise for out-of-range ids counted by deferred lookups (one sync)."""

    for device, counter in list(_DEFERRED_COUNTERS.items()):
        bad = int(counter.item())
        if bad:
            counter.zero_()
            raise IndexError(
                f"{bad} embedding lookups or bag poolings received out-of-range IDs "
                f"or inconsistent bag lengths on {device}"
            )


# ------------------------------------------------------------ plan types --


def embedding_local_bytes(
    *,
    rows: int,
    embedding_dim: int,
    weight_element_size: int,
    optimizer_state_layout: OptimizerStateLayout = "full",
) -> int:
    """Bytes of a local shard plus its sparse Adagrad state."""

    if rows < 0 or embedding_dim < 0 or weight_element_size <= 0:
        raise ValueError("rows, embedding_dim, and weight_element_size must be valid")
    weight_bytes = rows * embedding_dim * weight_element_size
    if optimizer_state_layout == "full":
        return weight_bytes + rows * embedding_dim * 4
    if optimizer_state_layout == "rowwise":
        return weight_bytes + rows * 4
    raise ValueError(
        f"optimizer_state_layout must be full or rowwise, got {optimizer_state_layout!r}"
    )


@dataclass(frozen=True)
class EmbeddingTableSpec:
    name: str
    num_embeddings: int
    embedding_dim: int
    element_size: int = 4

    @property
    def weight_bytes(self) -> int:
        return self.num_embeddings * self.embedding_dim * self.element_size


@dataclass(frozen=True)
class EmbeddingShardSpec:
    table_name: str
    strategy: EmbeddingShardStrategy
    world_size: int
    cyclic_offset: int = 0
    table_owner: int | None = None

    def owner(self, ids: Tensor) -> Tensor:
        if self.strategy == "row_wise":
            return torch.remainder(ids + self.cyclic_offset, self.world_size)
        if self.table_owner is None:
            raise RuntimeError("table-wise shard is missing its owner")
        return torch.full_like(ids, self.table_owner)

    def local_rows(self, num_embeddings: int, rank: int) -> int:
        if self.strategy == "table_wise":
            return num_embeddings if rank == self.table_owner else 0
        residue = (rank - self.cyclic_offset) % self.world_size
        if residue >= num_embeddings:
            return 0
        return (num_embeddings - 1 - residue) // self.world_size + 1

    def local_row_ids(self, global_ids: Tensor) -> Tensor:
        if self.strategy == "table_wise":
            return global_ids
        return torch.div(global_ids, self.world_size, rounding_mode="floor")


@dataclass(frozen=True)
class EmbeddingShardingPlan:
    world_size: int
    tables: dict[str, EmbeddingShardSpec]
    fingerprint: str


def _stable_offset(table_name: str, world_size: int) -> int:
    if world_size <= 1:
        return 0
    return int.from_bytes(sha256(table_name.encode("utf-8")).digest()[:8], "little") % world_size


def plan_embedding_shards(
    table_specs: Iterable[EmbeddingTableSpec],
    *,
    world_size: int,
    strategy: Literal["auto", "row_wise", "table_wise"],
    table_wise_max_rows: int,
    optimizer_state_layout: OptimizerStateLayout = "full",
) -> EmbeddingShardingPlan:
    """Deterministic placement: row-wise cyclic tables, then LPT for small ones.

    Same steps as src/embeddings.py:275-353, because what they produce is
    interface: the model reads ``plan.tables[name]`` to give each module its
    shard spec (src/model.py:2856-2859), checkpoints persist
    ``asdict(shard_spec)`` (src/checkpoint.py:447-464), and ``fingerprint``
    is a public field of the returned plan that only the same steps give.
    """

    if world_size <= 0:
        raise ValueError("world_size must be positive")
    if strategy not in {"auto", "row_wise", "table_wise"}:
        raise ValueError("strategy must be auto, row_wise, or table_wise")
    if optimizer_state_layout not in {"full", "rowwise"}:
        raise ValueError("optimizer_state_layout must be full or rowwise")
    specs = sorted(table_specs, key=lambda item: item.name)
    if len({item.name for item in specs}) != len(specs):
        raise ValueError("embedding table names must be unique")
    loads = [0] * world_size
    planned: dict[str, EmbeddingShardSpec] = {}
    small: list[EmbeddingTableSpec] = []
    for table in specs:
        if strategy == "table_wise" or (strategy == "auto" and table.num_embeddings <= table_wise_max_rows):
            small.append(table)
            continue
        shard = EmbeddingShardSpec(
            table_name=table.name,
            strategy="row_wise",
            world_size=world_size,
            cyclic_offset=_stable_offset(table.name, world_size),
        )
        planned[table.name] = shard
        for rank in range(world_size):
            loads[rank] += embedding_local_bytes(
                rows=shard.local_rows(table.num_embeddings, rank),
                embedding_dim=table.embedding_dim,
                weight_element_size=table.element_size,
                optimizer_state_layout=optimizer_state_layout,
            )
    for table in sorted(small, key=lambda item: (-item.weight_bytes, item.name)):
        owner = min(range(world_size), key=lambda rank: (loads[rank], rank))
        planned[table.name] = EmbeddingShardSpec(
            table_name=table.name, strategy="table_wise", world_size=world_size, table_owner=owner
        )
        loads[owner] += embedding_local_bytes(
            rows=table.num_embeddings,
            embedding_dim=table.embedding_dim,
            weight_element_size=table.element_size,
            optimizer_state_layout=optimizer_state_layout,
        )
    payload = {
        "world_size": world_size,
        "optimizer_state_layout": optimizer_state_layout,
        "cost_model_version": 2,
        "tables": {name: asdict(planned[name]) for name in sorted(planned)},
    }
    fingerprint = sha256(
        json.dumps(payload, sort_keys=True, separators=(",", ":")).encode("utf-8")
    ).hexdigest()
    return EmbeddingShardingPlan(world_size=world_size, tables=planned, fingerprint=fingerprint)


# ------------------------------------------------------------------ stats --


@dataclass
class EmbeddingCommunicationStats:
    table_name: str
    raw_ids: int = 0
    active_ids: int = 0
    local_unique_ids: int = 0
    owner_unique_ids: int = 0
    sent_ids: int = 0
    received_ids: int = 0
    forward_sent_bytes: int = 0
    forward_received_bytes: int = 0
    backward_sent_bytes: int = 0
    backward_received_bytes: int = 0
    forward_collective_enqueue_seconds: float = 0.0
    backward_collective_enqueue_seconds: float = 0.0

    @property
    def total_communication_bytes(self) -> int:
        return (
            self.forward_sent_bytes
            + self.forward_received_bytes
            + self.backward_sent_bytes
            + self.backward_received_bytes
        )

    def add_(self, other: "EmbeddingCommunicationStats") -> None:
        if self.table_name != other.table_name:
            raise ValueError("cannot combine communication stats for different tables")
        for name in (
            "raw_ids", "active_ids", "local_unique_ids", "owner_unique_ids", "sent_ids", "received_ids",
            "forward_sent_bytes", "forward_received_bytes", "backward_sent_bytes",
            "backward_received_bytes", "forward_collective_enqueue_seconds",
            "backward_collective_enqueue_seconds",
        ):
            setattr(self, name, getattr(self, name) + getattr(other, name))


class _EmbeddingStatsSink:
    def __init__(self, table_name: str) -> None:
        self.table_name = table_name
        self._stats = EmbeddingCommunicationStats(table_name=table_name)

    def record_forward(self, stats: EmbeddingCommunicationStats) -> None:
        self._stats.add_(stats)

    def consume(self) -> EmbeddingCommunicationStats:
        result = self._stats
        self._stats = EmbeddingCommunicationStats(table_name=self.table_name)
        return result


def _local_stats(table_name: str, raw_ids: int) -> EmbeddingCommunicationStats:
    # Single-rank lookups move nothing; unique counts are not measured (no sync).
    return EmbeddingCommunicationStats(
        table_name=table_name, raw_ids=raw_ids, active_ids=raw_ids,
        local_unique_ids=raw_ids, owner_unique_ids=raw_ids,
    )


def _distributed_rank_world(process_group: Any) -> tuple[int, int]:
    if not torch_dist.is_available() or not torch_dist.is_initialized():
        return 0, 1
    return torch_dist.get_rank(process_group), torch_dist.get_world_size(process_group)


# ------------------------------------------------------------- autograd --


def _raise_for_errors(modules: list["ShardedEmbedding"], ids: list[Tensor], err: Tensor) -> None:
    """Reference error behaviour: IndexError naming the table and examples."""

    if not int(err.reshape(-1)[0].item()):
        return
    for module, t in zip(modules, ids):
        flat = t.reshape(-1)
        invalid = (flat < 0) | (flat >= module.num_embeddings)
        if bool(invalid.any()):
            examples = flat[invalid][:5].detach().cpu().tolist()
            raise IndexError(
                f"embedding {module.table_name!r} received IDs outside "
                f"[0, {module.num_embeddings}): {examples}"
            )
    raise IndexError("embedding lookup received out-of-range IDs")


def _check_ids(modules: list["ShardedEmbedding"], ids: list[Tensor], err: Tensor) -> None:
    checked = [m for m in modules if m.validate_indices]
    if not checked:
        return
    if err.device.type != "cuda":
        _raise_for_errors(modules, ids, err)
        return
    mode = index_check_mode()
    if mode == "sync":
        _raise_for_errors(modules, ids, err)
    elif mode == "deferred":
        _deferred_counter(err.device).add_(err.reshape(-1)[:1])
    else:
        names = ", ".join(repr(m.table_name) for m in checked[:4])
        torch._assert_async(err == 0, f"embedding {names} received an out-of-range ID")


_POOLING_CODES = {"none": 0, "sum": 1, "mean": 2}


def _grouped_lookup(
    modules: list["ShardedEmbedding"],
    ids: list[Tensor],
    lengths: list[Tensor | None],
    poolings: list[str],
    null_policies: list[str],
) -> list[Tensor]:
    """One ``mdl_hip::grouped_lookup`` call for every request; requests on
    the same module share its table (one coalesced gradient per table)."""

    weights: list[Tensor] = []
    index: dict[int, int] = {}
    table, codes, exclude, padding = [], [], [], []
    # one pass over the requests: each table once, and the per-feature codes
    for module, pooling, policy in zip(modules, poolings, null_policies):
        w = module.weight
        t = index.get(id(w))
        if t is None:
            t = index[id(w)] = len(weights)
            weights.append(w)
        table.append(t)
        codes.append(_POOLING_CODES[pooling])
        if policy == "exclude":
            exclude.append(1)
        elif policy == "include_as_padding":
            exclude.append(0)
        else:
            raise ValueError(f"unsupported categorical bag null policy {policy!r}")
        padding.append(int(module.padding_idx))
    need_backward = torch.is_grad_enabled() and any(w.requires_grad for w in weights)
    spec = (table, codes, exclude, padding)
    ids = list(ids)
    if need_backward:
        # one autograd node in C++ over the tables (no Python in the
        # backward); tracers get the op's registered autograd instead
        *outputs, err = torch.ops.mdl_hip.grouped_lookup_autograd(weights, ids, list(lengths), *spec)
    else:
        outputs, _, _, _, _, err = torch.ops.mdl_hip.grouped_lookup_untracked(weights, ids, list(lengths), *spec,
                                                                              False)
    _check_ids(modules, ids, err)
    return list(outputs)


# ----------------------------------------------------------------- module --


class ShardedEmbedding(nn.Module):
    """``nn.Embedding``-compatible table with a HIP lookup and sparse grads."""

    def __init__(
        self,
        num_embeddings: int,
        embedding_dim: int,
        *,
        table_name: str,
        shard_spec: EmbeddingShardSpec,
        padding_idx: int = 0,
        local_dedup: bool = True,
        init_std: float = 0.02,
        process_group: Any = None,
        dtype: torch.dtype | None = None,
        collect_stats: bool = True,
        validate_indices: bool = True,
    ) -> None:
        super().__init__()
        if num_embeddings <= 0 or embedding_dim <= 0:
            raise ValueError("num_embeddings and embedding_dim must be positive")
        if not 0 <= padding_idx < num_embeddings:
            raise ValueError("padding_idx must be inside the embedding table")
        rank, world_size = _distributed_rank_world(process_group)
        if world_size != shard_spec.world_size:
            raise ValueError("shard spec world size does not match the active process group")
        self.num_embeddings = num_embeddings
        self.embedding_dim = embedding_dim
        self.padding_idx = padding_idx
        self.sparse = True
        self.table_name = table_name
        self.shard_spec = shard_spec
        self.local_dedup = local_dedup
        self.init_std = init_std
        self.process_group = process_group
        self.collect_stats = collect_stats
        self.validate_indices = validate_indices
        self.rank = rank
        self.world_size = world_size
        local_rows = shard_spec.local_rows(num_embeddings, rank)
        self.weight = nn.Parameter(torch.empty(local_rows, embedding_dim, dtype=dtype))
        self._stats_sink = _EmbeddingStatsSink(table_name)
        self.reset_parameters()

    def reset_parameters(self) -> None:
        table_seed = int.from_bytes(sha256(self.table_name.encode("utf-8")).digest()[:8], "little")
        seed = (torch.initial_seed() + table_seed + self.rank * 104729) % (2**63 - 1)
        generator = torch.Generator(device=self.weight.device)
        generator.manual_seed(seed)
        nn.init.normal_(self.weight, mean=0.0, std=self.init_std, generator=generator)
        if self.shard_spec.strategy == "table_wise":
            padding_owner = self.shard_spec.table_owner
            local_padding = self.padding_idx
        else:
            padding_owner = (self.padding_idx + self.shard_spec.cyclic_offset) % self.world_size
            local_padding = self.padding_idx // self.world_size
        if padding_owner == self.rank:
            with torch.no_grad():
                self.weight[local_padding].zero_()

    def _require_single_rank(self) -> None:
        if self.world_size != 1:
            raise NotImplementedError(
                "multi-GPU owner routing is not part of the single-GPU MI355X build"
            )

    def forward(self, indices: Tensor) -> Tensor:
        self._require_single_rank()
        if indices.dtype != torch.long:
            raise TypeError("sharded embedding indices must be torch.long")
        output = _grouped_lookup([self], [indices], [None], ["none"], ["include_as_padding"])[0]
        if self.collect_stats and embedding_stats_host_sync_enabled():
            self._stats_sink.record_forward(_local_stats(self.table_name, int(indices.numel())))
        return output

    @torch.no_grad()
    def load_full_weight_(self, full_weight: Tensor) -> None:
        """Load a full table (tests and migration tools)."""

        expected = (self.num_embeddings, self.embedding_dim)
        if tuple(full_weight.shape) != expected:
            raise ValueError(f"full weight must have shape {expected}")
        global_ids = torch.arange(self.num_embeddings, dtype=torch.long, device=full_weight.device)
        owned = self.shard_spec.owner(global_ids) == self.rank
        local_values = full_weight.index_select(0, global_ids[owned])
        if tuple(local_values.shape) != tuple(self.weight.shape):
            raise RuntimeError("full weight slice does not match local shard shape")
        self.weight.copy_(local_values.to(device=self.weight.device, dtype=self.weight.dtype))

    def consume_communication_stats(self) -> EmbeddingCommunicationStats:
        return self._stats_sink.consume()

    def extra_repr(self) -> str:
        return (
            f"num_embeddings={self.num_embeddings}, embedding_dim={self.embedding_dim}, "
            f"local_rows={self.weight.size(0)}, strategy={self.shard_spec.strategy}, "
            f"rank={self.rank}/{self.world_size}, padding_idx={self.padding_idx}, "
            f"validate_indices={self.validate_indices}"
        )


def grouped_sharded_embedding_lookup(
    requests: Iterable[tuple[ShardedEmbedding, Tensor]],
    *,
    max_output_bytes: int | None = None,
) -> list[Tensor]:
    """Look up many (module, ids) requests in one launch.

    ``max_output_bytes`` bounds the reference's multi-GPU exchange buffers;
    a single-GPU lookup has none, so it is only validated.
    """

    request_list = list(requests)
    if not request_list:
        return []
    if max_output_bytes is not None and int(max_output_bytes) <= 0:
        raise ValueError("grouped embedding max output bytes must be positive")
    modules, ids = [], []
    for module, t in request_list:
        if module.world_size != 1:
            module._require_single_rank()
        if t.dtype != torch.long:
            raise TypeError("sharded embedding indices must be torch.long")
        modules.append(module)
        ids.append(t)
    outputs = _grouped_lookup(
        modules, ids, [None] * len(ids), ["none"] * len(ids), ["include_as_padding"] * len(ids)
    )
    if embedding_stats_host_sync_enabled():
        for module, t in request_list:
            if module.collect_stats:
                module._stats_sink.record_forward(_local_stats(module.table_name, int(t.numel())))
    return outputs


def pooled_embedding_lookup(
    requests: Iterable[tuple[ShardedEmbedding, Tensor, Tensor, str, str]],
) -> list[Tensor]:
    """Fused lookup + bag pooling of many features in one launch.

    Each request is ``(module, values, lengths, pooling, null_policy)`` with
    CSR ``values`` [sum(lengths)] and ``lengths`` [B]; ``pooling`` is ``mean``
    (src/model.py:509-678) or ``sum``.  Returns one ``[B, dim]`` tensor per
    request -- the same numbers as ``module(values)`` followed by
    ``_mean_pool_categorical_bag``, without materialising the per-id rows.
    """

    request_list = list(requests)
    if not request_list:
        return []
    for module, values, lengths, pooling, policy in request_list:
        if module.world_size != 1:
            module._require_single_rank()
        if pooling not in ("mean", "sum"):
            raise ValueError("pooled lookups use mean or sum pooling")
        if lengths.ndim != 1:
            raise ValueError("categorical bag lengths must have shape [B]")
    return _grouped_lookup(
        [r[0] for r in request_list],
        [r[1] for r in request_list],
        [r[2] for r in request_list],
        [r[3] for r in request_list],
        [r[4] for r in request_list],
    )


def sequence_embedding_lookup(
    module: ShardedEmbedding,
    ids: Tensor,
    lengths: Tensor,
    *,
    target_length: int | None = None,
    sequence_order: str = "oldest_to_newest",
) -> tuple[Tensor, Tensor]:
    """Embed a right-padded ``[B, L]`` id sequence into a right-aligned window.

    Same result as ``module(ids)`` followed by ``_right_aligned_sequence`` (and
    the reversal of ``_align_sequence_inputs`` for ``newest_to_oldest``),
    src/model.py:2989-3100: ``([B, T, dim] embeddings, [B, T] bool mask)`` with
    ``T = target_length or L``; the padded window is written in one launch.
    """

    module._require_single_rank()
    if ids.dtype != torch.long:
        raise TypeError("sharded embedding indices must be torch.long")
    if ids.ndim != 2 or lengths.ndim != 1 or lengths.numel() != ids.size(0):
        raise ValueError("sequence ids must be [B, L] with lengths [B]")
    if sequence_order not in ("oldest_to_newest", "newest_to_oldest"):
        raise ValueError("sequence_order must be oldest_to_newest or newest_to_oldest")
    w = module.weight
    need_backward = torch.is_grad_enabled() and w.requires_grad
    out, mask, _, _, err = torch.ops.mdl_hip.sequence_lookup(
        w, ids, lengths.to(device=ids.device, dtype=torch.int64), int(ids.size(1) if target_length is None
                                                                      else target_length),
        sequence_order == "newest_to_oldest", int(module.padding_idx), need_backward,
    )
    _check_ids([module], [ids], err)
    if module.collect_stats and embedding_stats_host_sync_enabled():
        module._stats_sink.record_forward(_local_stats(module.table_name, int(ids.numel())))
    return out, mask


def sharded_embedding_modules(module: nn.Module) -> list[ShardedEmbedding]:
    return [item for item in module.modules() if isinstance(item, ShardedEmbedding)]


def consume_sharded_embedding_stats(module: nn.Module) -> list[EmbeddingCommunicationStats]:
    return [
        item.consume_communication_stats()
        for item in sharded_embedding_modules(module)
        if item.collect_stats
    ]
