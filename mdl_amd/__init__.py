"""MI355X (gfx950) sparse-feature path of an MDL/RankMixer-style ranker.

Hashed multi-value embedding-bag lookup, its deterministic sort/unique/
segment-reduce backward and the row-wise Adagrad update, as hand-written HIP
kernels in ``libmdl_hip.so`` behind the reference's Python API:

* :mod:`mdl_amd.embeddings` -- ``ShardedEmbedding``, ``grouped_sharded_embedding_lookup``,
  ``pooled_embedding_lookup`` and the sharding-plan types;
* :mod:`mdl_amd.optim` -- ``ShardedRowWiseAdagrad``, ``fused_rowwise_adagrad_update``;
* :mod:`mdl_amd.features` -- ``pre_hashed`` / ``mod`` bucketing and CSR bags;
* :mod:`mdl_amd.pooling` -- the pooling helpers of the encoder bank;
* :mod:`mdl_amd.sparse_step` -- one fused forward + backward + update step;
* :mod:`mdl_amd.ops` -- tensor-level calls of the C ABI (include/mdl_hip.h);
* :mod:`mdl_amd.library` -- the same path as ``torch.library`` custom ops
  (``torch.ops.mdl_hip.*``, registered when the package is imported).
"""

from . import library  # noqa: F401  (registers the mdl_hip ops)
from ._lib import LIB_PATH, MdlError, lib

__all__ = ["LIB_PATH", "MdlError", "lib"]
