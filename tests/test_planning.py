"""Host logic of the drop-in embedding API on CPU, written like the
reference's own tests: shard planning and its fingerprint
(tests/test_sharded_embedding.py:596-646), the local-bytes cost model
(tests/test_rowwise_adagrad.py:174-213) and the per-table lookup statistics
(src/embeddings.py:26-59,813-814,1754-1765), row ownership and the
communication-stats record (src/embeddings.py:163-188,198-240)."""

import pytest
import torch
from torch import nn

from mdl_amd.embeddings import (
    EmbeddingCommunicationStats,
    EmbeddingTableSpec,
    ShardedEmbedding,
    consume_sharded_embedding_stats,
    embedding_local_bytes,
    embedding_stats_host_sync,
    grouped_sharded_embedding_lookup,
    plan_embedding_shards,
    set_embedding_stats_host_sync,
    sharded_embedding_modules,
)


def test_embedding_local_bytes_formulas():
    assert embedding_local_bytes(rows=1000, embedding_dim=64, weight_element_size=2,
                                 optimizer_state_layout="full") == 1000 * 64 * (2 + 4)
    assert embedding_local_bytes(rows=1000, embedding_dim=64, weight_element_size=2,
                                 optimizer_state_layout="rowwise") == 1000 * (64 * 2 + 4)


def test_plan_default_layout_is_full_and_rowwise_changes_fingerprint():
    specs = [EmbeddingTableSpec(name="a", num_embeddings=100, embedding_dim=8, element_size=2),
             EmbeddingTableSpec(name="b", num_embeddings=50, embedding_dim=4, element_size=2)]
    full = plan_embedding_shards(specs, world_size=2, strategy="row_wise", table_wise_max_rows=1)
    rowwise = plan_embedding_shards(specs, world_size=2, strategy="row_wise", table_wise_max_rows=1,
                                    optimizer_state_layout="rowwise")
    assert full.fingerprint != rowwise.fingerprint


def test_auto_uses_row_wise_for_large_and_lpt_for_small_tables():
    specs = [EmbeddingTableSpec("large", 1000, 8), EmbeddingTableSpec("small_a", 20, 8),
             EmbeddingTableSpec("small_b", 10, 8)]
    first = plan_embedding_shards(specs, world_size=2, strategy="auto", table_wise_max_rows=32)
    second = plan_embedding_shards(reversed(specs), world_size=2, strategy="auto", table_wise_max_rows=32)
    assert first.fingerprint == second.fingerprint
    assert first.tables["large"].strategy == "row_wise"
    assert first.tables["small_a"].strategy == "table_wise"
    assert first.tables["small_a"].table_owner != first.tables["small_b"].table_owner


def test_rowwise_cost_model_matches_embedding_local_bytes():
    plan = plan_embedding_shards([EmbeddingTableSpec("t0", 1000, 64, element_size=2)], world_size=2,
                                 strategy="row_wise", table_wise_max_rows=1, optimizer_state_layout="rowwise")
    shard = plan.tables["t0"]
    assert sum(shard.local_rows(1000, rank) for rank in range(2)) == 1000
    for rank in range(2):
        rows = shard.local_rows(1000, rank)
        assert embedding_local_bytes(rows=rows, embedding_dim=64, weight_element_size=2,
                                     optimizer_state_layout="rowwise") == rows * (64 * 2 + 4)


def _model():
    plan = plan_embedding_shards([EmbeddingTableSpec("a", 16, 4), EmbeddingTableSpec("b", 12, 4)], world_size=1,
                                 strategy="row_wise", table_wise_max_rows=32)
    model = nn.ModuleDict({
        "a": ShardedEmbedding(16, 4, table_name="a", shard_spec=plan.tables["a"]),
        "b": ShardedEmbedding(12, 4, table_name="b", shard_spec=plan.tables["b"], collect_stats=False),
    })
    return model


def test_lookup_statistics_are_recorded_and_consumed():
    model = _model()
    assert [m.table_name for m in sharded_embedding_modules(model)] == ["a", "b"]
    model["a"](torch.tensor([1, 2, 3]))
    grouped_sharded_embedding_lookup([(model["a"], torch.tensor([[4, 5], [0, 6]])), (model["b"], torch.tensor([7]))])
    stats = consume_sharded_embedding_stats(model)
    # only tables that collect statistics report; a single-GPU lookup moves nothing
    assert [s.table_name for s in stats] == ["a"]
    assert stats[0].raw_ids == 7 and stats[0].active_ids == 7 and stats[0].sent_ids == 0
    assert consume_sharded_embedding_stats(model)[0].raw_ids == 0  # consumed
    with embedding_stats_host_sync(False):
        model["a"](torch.tensor([1, 2]))
    assert consume_sharded_embedding_stats(model)[0].raw_ids == 0


def test_table_initialisation_matches_the_reference_bit_for_bit():
    """Golden weights written by the reference's own ShardedEmbedding
    (tests/golden/make_init_vectors.py): the seed from torch.initial_seed(),
    the table name's sha256 and the rank, N(0, init_std), the padding row
    zeroed -- so a checkpoint-free run starts from the reference's tables."""

    import json
    import pathlib

    cases = json.loads((pathlib.Path(__file__).parent / "golden" / "init_vectors.json").read_text())
    assert cases
    for c in cases:
        plan = plan_embedding_shards([EmbeddingTableSpec(c["name"], c["rows"], c["dim"])], world_size=1,
                                     strategy="row_wise", table_wise_max_rows=1)
        torch.manual_seed(c["seed"])
        m = ShardedEmbedding(c["rows"], c["dim"], table_name=c["name"], shard_spec=plan.tables[c["name"]],
                             padding_idx=c["padding_idx"], init_std=c["init_std"], dtype=getattr(torch, c["dtype"]),
                             collect_stats=False)
        expect = torch.tensor(c["weight"], dtype=torch.float32).to(getattr(torch, c["dtype"]))
        assert torch.equal(m.weight.detach(), expect), c["name"]
        assert not m.weight[c["padding_idx"]].any()


def test_row_ownership_and_local_row_ids():
    """Row-wise shards own ``(id + offset) mod W`` and store row ``id div W``;
    a table-wise shard owns every id at its global row (src/embeddings.py:163-188)."""

    plan = plan_embedding_shards([EmbeddingTableSpec("big", 1000, 8), EmbeddingTableSpec("small", 10, 8)],
                                 world_size=3, strategy="auto", table_wise_max_rows=100)
    big, small = plan.tables["big"], plan.tables["small"]
    assert big.strategy == "row_wise" and small.strategy == "table_wise"
    ids = torch.arange(0, 20)
    owners = big.owner(ids)
    assert torch.equal(owners, (ids + big.cyclic_offset) % 3)
    assert torch.equal(big.local_row_ids(ids), ids // 3)
    # every global row has exactly one (owner, local row), and each owner's
    # local rows fill [0, local_rows) without gaps
    all_ids = torch.arange(1000)
    o, local = big.owner(all_ids), big.local_row_ids(all_ids)
    for rank in range(3):
        mine = local[o == rank]
        assert mine.numel() == big.local_rows(1000, rank)
        assert torch.equal(mine.sort().values, torch.arange(mine.numel()))
    assert torch.equal(small.owner(ids), torch.full_like(ids, small.table_owner))
    assert torch.equal(small.local_row_ids(ids), ids)
    assert [small.local_rows(10, r) for r in range(3)] == [10 if r == small.table_owner else 0 for r in range(3)]


def test_communication_stats_add_up():
    a = EmbeddingCommunicationStats("t", raw_ids=5, forward_sent_bytes=10, backward_received_bytes=3)
    b = EmbeddingCommunicationStats("t", raw_ids=2, forward_received_bytes=7, backward_sent_bytes=1)
    a.add_(b)
    assert a.raw_ids == 7 and a.total_communication_bytes == 21
    with pytest.raises(ValueError, match="different tables"):
        a.add_(EmbeddingCommunicationStats("u"))


def test_stats_host_sync_switch_is_thread_local_and_restored():
    import threading

    set_embedding_stats_host_sync(False)
    try:
        model = _model()
        model["a"](torch.tensor([1, 2, 3]))
        assert consume_sharded_embedding_stats(model)[0].raw_ids == 0  # no host reads, nothing counted
        seen = []
        t = threading.Thread(target=lambda: seen.append(_host_sync_enabled()))
        t.start()
        t.join()
        assert seen == [True]  # another thread keeps the default
        with embedding_stats_host_sync(True):
            model["a"](torch.tensor([1, 2, 3]))
        assert consume_sharded_embedding_stats(model)[0].raw_ids == 3
        assert not _host_sync_enabled()  # restored
    finally:
        set_embedding_stats_host_sync(True)


def _host_sync_enabled():
    from mdl_amd import embeddings

    return getattr(embeddings._STATS_HOST_SYNC, "enabled", True)
