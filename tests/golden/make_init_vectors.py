"""Golden vectors of the reference's embedding-table initialisation, which
no test of the reference pins: src/embeddings.py:723-749 seeds a generator
from torch.initial_seed(), the first 8 bytes of the table name's sha256 and
the rank, draws N(0, init_std) and zeroes the padding row.

Run once where the reference tree is present (not on the GPU box):
    python tests/golden/make_init_vectors.py /root/reference
It writes init_vectors.json beside this script; the tests read only that."""

import json
import pathlib
import sys

import torch

CASES = [
    # (torch seed, table name, rows, dim, init std, padding_idx, dtype)
    (0, "user_id", 6, 4, 0.02, 0, "float32"),
    (1234, "item_id", 5, 8, 0.02, 2, "float32"),
    (7, "table_17", 4, 3, 0.5, 3, "float32"),
    (99, "cate", 3, 16, 0.02, 0, "bfloat16"),
]


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from src.embeddings import EmbeddingTableSpec, ShardedEmbedding, plan_embedding_shards

    out = []
    for seed, name, rows, dim, std, pad, dtype in CASES:
        plan = plan_embedding_shards([EmbeddingTableSpec(name, rows, dim)], world_size=1, strategy="row_wise",
                                     table_wise_max_rows=1)
        torch.manual_seed(seed)
        m = ShardedEmbedding(rows, dim, table_name=name, shard_spec=plan.tables[name], padding_idx=pad,
                             init_std=std, dtype=getattr(torch, dtype), collect_stats=False)
        out.append({"seed": seed, "name": name, "rows": rows, "dim": dim, "init_std": std, "padding_idx": pad,
                    "dtype": dtype, "weight": m.weight.detach().float().tolist()})
    path = pathlib.Path(__file__).with_name("init_vectors.json")
    path.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {len(out)} cases to {path}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
