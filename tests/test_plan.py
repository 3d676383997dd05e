"""Key groups of a grouped plan (host logic, no GPU).

A plan of 2^32 - 1 rows or more is cut into runs of consecutive features whose
tables share one 32-bit key space.  The tables here are stride-0 views of a
one-row tensor: only their row counts matter to the cut.
"""

import numpy as np
import pytest
import torch

from mdl_amd import library, ops


def _plan(rows, feature_tables, pooling=None):
    plan = ops.GroupPlan()
    for r in rows:
        plan.tables.append(ops.TableSpec(weight=torch.zeros(1, 8).expand(int(r), 8), state=None,
                                         row_base=plan.total_rows))
        plan.total_rows += int(r)
    for f, t in enumerate(feature_tables):
        plan.features.append(ops.FeatureSpec(table=t, pooling=0 if pooling is None else pooling[f],
                                             exclude_null=True, padding_idx=0, out_dtype=torch.bfloat16))
    return plan


def _check_invariants(plan):
    groups = plan.groups
    assert groups[0].lo == 0 and groups[-1].hi == len(plan.features)
    seen = set()
    for a, b in zip(groups, groups[1:]):
        assert a.hi == b.lo
    for g in groups:
        assert g.rows < ops.KEY_SPACE
        assert g.rows == sum(int(plan.tables[t].weight.size(0)) for t in g.tables)
        # the group's tables tile [0, rows) of its key space
        spans = sorted((plan.tables[t].row_base, int(plan.tables[t].weight.size(0))) for t in g.tables)
        end = 0
        for base, r in spans:
            assert base == end
            end += r
        assert end == g.rows
        for f in range(g.lo, g.hi):
            assert plan.features[f].table in g.tables
        assert not seen & set(g.tables)
        seen |= set(g.tables)
        # the group as a plan of its own: same specs, tables renumbered
        assert [plan.tables[t] for t in g.tables] == g.plan.tables
        for f, sub in zip(range(g.lo, g.hi), g.plan.features):
            assert g.tables[sub.table] == plan.features[f].table
            assert sub.pooling == plan.features[f].pooling
        assert g.plan.groups[0].rows == g.rows and not g.plan.split
    assert plan.sentinel == max(g.rows for g in groups)
    assert plan.key_bits == int(plan.sentinel).bit_length() <= 32


def test_plan_below_key_space_is_one_group():
    plan = _plan([10, 2_000_000_000, 7], [1, 0, 2, 1])
    assert not plan.split
    (g,) = plan.groups
    assert (g.lo, g.hi, g.tables, g.rows) == (0, 4, [0, 1, 2], 2_000_000_017)
    assert [t.row_base for t in plan.tables] == [0, 10, 2_000_000_010]
    assert plan.sentinel == 2_000_000_017
    _check_invariants(plan)


def test_plan_of_4_5e9_rows_cuts_two_key_groups():
    rows = [2_200_000_000, 2_300_000_000, 10_000]
    plan = _plan(rows, [0, 0, 1, 2], pooling=[2, 0, 1, 0])
    assert plan.split
    g0, g1 = plan.groups
    assert (g0.lo, g0.hi, g0.tables, g0.rows) == (0, 2, [0], 2_200_000_000)
    assert (g1.lo, g1.hi, g1.tables, g1.rows) == (2, 4, [1, 2], 2_300_010_000)
    assert [t.row_base for t in plan.tables] == [0, 0, 2_300_000_000]
    assert plan.sentinel == 2_300_010_000 and plan.key_bits == 32
    _check_invariants(plan)


def test_plan_rereading_a_closed_group_is_refused():
    plan = _plan([2_200_000_000, 2_300_000_000], [0, 1, 0])
    with pytest.raises(ValueError, match="table 0 is read again by feature 2"):
        plan.groups


def test_plan_key_groups_on_random_layouts():
    rng = np.random.default_rng(7)
    for _ in range(200):
        T = int(rng.integers(1, 12))
        rows = rng.integers(1, 3_000_000_000, size=T)
        tables = np.sort(rng.integers(0, T, size=int(rng.integers(1, 30))))
        plan = _plan(rows, [int(t) for t in tables])
        _check_invariants(plan)
        used = sorted(set(int(t) for t in tables))
        assert plan.split == (int(rows.sum()) >= ops.KEY_SPACE and len(plan.groups) > 1)
        # past the key space the groups key the tables the features read;
        # below it, one group keys every table
        expect = used if int(rows.sum()) >= ops.KEY_SPACE else list(range(T))
        assert sorted(t for g in plan.groups for t in g.tables) == expect


def test_grouped_lookup_orders_features_by_table_past_the_key_space():
    small = [torch.zeros(1, 8).expand(10, 8), torch.zeros(1, 8).expand(20, 8)]
    assert library._order(small, [1, 0, 1]) is None
    big = [torch.zeros(1, 8).expand(2_200_000_000, 8), torch.zeros(1, 8).expand(2_300_000_000, 8)]
    assert library._order(big, [0, 1, 0]) == [0, 2, 1]
    assert library._order(big, [0, 0, 1]) is None
    order = library._order(big, [1, 0, 1, 0])
    assert order == [1, 3, 0, 2]
    plan = _plan([2_200_000_000, 2_300_000_000], [[1, 0, 1, 0][f] for f in order])
    _check_invariants(plan)
