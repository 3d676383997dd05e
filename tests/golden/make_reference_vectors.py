"""Write reference_vectors.json: the hot-path golden vectors that the
reference's own unit tests hold, transcribed as data with their sources.

Every entry is an input/expected-output pair copied from a reference test
file (path:line given in "source"); nothing here runs reference code.
Run: python tests/golden/make_reference_vectors.py
"""

import json
from pathlib import Path

INT64_MIN = -(1 << 63)
INT64_MAX = (1 << 63) - 1

VECTORS = {
    "pre_hashed_scalar": {
        "source": "tests/test_direct_id.py:183-189",
        "num_buckets": 8,
        "cases": [[-1, 8], [-8, 1], [INT64_MIN, 1], [INT64_MAX, 8]],
        "zero_raises": True,
    },
    "pre_hashed_column_with_nulls": {
        "source": "tests/test_direct_id.py:191-212",
        "num_buckets": 8,
        "raw": [None, -1, -8, INT64_MIN, 1, INT64_MAX],
        "expected": [0, 8, 1, 1, 2, 8],
    },
    "pre_hashed_zero_unvalidated": {
        "source": "tests/test_direct_id.py:224-240",
        "num_buckets": 8,
        "raw": [1, 0],
        "expected": [2, 1],
    },
    "pre_hashed_sequence_head": {
        "source": "tests/test_direct_id.py:242-280",
        "num_buckets": 8,
        "rows": [[-1, -8, 3], None],
        "max_length": 2,
        "truncation": "head",
        "expected_lengths": [2, 0],
        "expected_padded": [[8, 1], [0, 0]],
    },
    "bag_head_truncation": {
        "source": "tests/test_multivalue_features.py:38-66",
        "num_buckets": 8,
        "rows": [[1, None, -1, 4], None, [-8]],
        "max_length": 3,
        "truncation": "head",
        "expected_lengths": [3, 0, 1],
        "expected_values": [2, 0, 8, 1],
    },
    "bag_tail_truncation": {
        "source": "tests/test_multivalue_features.py:68-93",
        "num_buckets": 8,
        "rows": [[1, None, -1, 4], [7], [-8, 3, 5, 9]],
        "max_length": 3,
        "truncation": "tail",
        "expected_lengths": [3, 1, 3],
        "expected_values": [0, 8, 5, 8, 4, 6, 2],
    },
    "mean_pool_null_policies": {
        "source": "tests/test_multivalue_features.py:95-111",
        "indices": [2, 0, 8],
        "lengths": [3, 0],
        "embedded_is_index_value": True,
        "expected_exclude": [[5.0], [0.0]],
        "expected_include_as_padding": [[10.0 / 3.0], [0.0]],
    },
    "mean_pool_padded": {
        "source": "tests/test_multivalue_features.py:113-121",
        "indices": [[2, 0, 8], [0, 0, 0]],
        "lengths": [3, 0],
        "embedded_is_index_value": True,
        "expected_exclude": [[5.0], [0.0]],
    },
    "rowwise_adagrad_mean_not_sum": {
        "source": "tests/test_rowwise_adagrad.py:40-62",
        "shape": [4, 2],
        "lr": 0.5,
        "eps": 1e-8,
        "acc0": 0.0,
        "rows": [1, 3],
        "values": [[2.0, 0.0], [1.0, -1.0]],
        "expected_acc": {"1": 2.0, "3": 1.0},
        "expected_neg_weight": {
            "1": [2.0 / (2.0 ** 0.5 + 1e-8) * 0.5, 0.0],
            "3": [1.0 / (1.0 + 1e-8) * 0.5, -1.0 / (1.0 + 1e-8) * 0.5],
        },
        "atol": 1e-6,
    },
    "rowwise_adagrad_duplicates_coalesce": {
        "source": "tests/test_rowwise_adagrad.py:64-81",
        "shape": [5, 2],
        "lr": 1.0,
        "eps": 1e-8,
        "rows": [3, 3, 3],
        "values": [[1.0, 0.0], [1.0, 0.0], [1.0, 0.0]],
        "expected_acc": {"3": 4.5},
        "expected_nonzero_acc_rows": 1,
    },
    "rowwise_adagrad_empty_noop": {
        "source": "tests/test_rowwise_adagrad.py:83-100",
        "shape": [3, 2],
        "lr": 0.1,
        "acc0": 0.25,
        "expected_step": 1.0,
    },
    "rowwise_adagrad_bf16_untouched": {
        "source": "tests/test_rowwise_adagrad.py:102-128",
        "weight": [[0, 1], [2, 3], [4, 5], [6, 7]],
        "lr": 0.25,
        "eps": 1e-8,
        "rows": [1, 1],
        "values": [[1.0, -1.0], [1.0, 1.0]],
        "expected_acc_row1": 2.0,
        "untouched_rows": [0, 2, 3],
    },
    "rowwise_adagrad_shard_vs_full": {
        "source": "tests/test_sharded_embedding.py:647-699",
        "note": "full-table rows [0,3,5] with these grads; weights from torch.manual_seed(0) randn(8,4) in the reference test; here the weights are any fixed table and the check is shard-vs-full equality",
        "rows": [0, 3, 5],
        "values": [[1.0, 0.0, -1.0, 0.5], [0.5, 0.5, 0.0, 0.0], [2.0, 0.0, 0.0, 1.0]],
        "lr": 0.1,
        "eps": 1e-8,
    },
    "embedding_local_bytes": {
        "source": "tests/test_rowwise_adagrad.py:174-192",
        "rows": 1000,
        "dim": 64,
        "element_size": 2,
        "full": 1000 * 64 * (2 + 4),
        "rowwise": 1000 * (64 * 2 + 4),
    },
}

if __name__ == "__main__":
    out = Path(__file__).with_name("reference_vectors.json")
    out.write_text(json.dumps(VECTORS, indent=1, sort_keys=True) + "\n")
    print(out)
