"""bench.py's algorithmic byte count on hand-counted workloads (CPU only).

The per-step figure follows the pooled formula
sum over tables of 16 n_t + 16 (b_t + 1) + 3 U_t D_t s_w + 8 U_t, plus
2 B D_f s_o per feature, with the pooled output and its gradient counted at
the element size of the buffers the bench allocates (the tables' dtype), and
padding ids (0) not counted as looked up."""

import sys
from pathlib import Path

import numpy as np
import pytest

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
import bench  # noqa: E402


def _workload(dtype):
    feats = [bench.Feature(table=0, pooling="mean", bag_len=(1, 4)),
             bench.Feature(table=1, pooling="none", bag_len=None),
             bench.Feature(table=0, pooling="sum", bag_len=(1, 4))]
    return bench.Workload(name="t", batch=3, rows=[100, 50], dims=[16, 8], dtype=dtype, features=feats,
                          zipf=[0.0, 0.0])


@pytest.mark.parametrize("dtype,size", [("fp32", 4), ("bf16", 2)])
def test_pooled_bytes_are_the_hand_count(dtype, size):
    wl = _workload(dtype)
    ids = [np.array([5, 7, 5, 0, 9]), np.array([3, 3, 4]), np.array([7, 11])]
    lengths = [np.array([2, 1, 2]), None, np.array([1, 0, 1])]
    got = bench.algorithmic_bytes(wl, ids, lengths)
    # table 0: ids 5 7 5 9 7 11 (the 0 is padding) -> n 6, U 4 (5 7 9 11), bags 3 + 3
    # table 1: ids 3 3 4 -> n 3, U 2, one pseudo-bag per row (3)
    t0 = 16 * 6 + 16 * (6 + 1) + 3 * 4 * 16 * size + 8 * 4
    t1 = 16 * 3 + 16 * (3 + 1) + 3 * 2 * 8 * size + 8 * 2
    outputs = 2 * 3 * (16 + 8 + 16) * size
    assert got["B_alg"] == t0 + t1 + outputs
    assert got["n_ids"] == 9 and got["unique_rows"] == 6 and got["sum_dim"] == 40
