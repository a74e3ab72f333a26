"""Indexer -> sparse attention on one packed (TND) batch: the DSA prefill step.

The reference chains its two entry points by hand: ``lightning_indexer_triton``
(lightning_indexer_triton.py:466-554) returns the per-row top-k positions, which
go straight into ``sparse_flash_attention_triton`` (sparse_flash_attention_triton.py:1295-1455)
as ``sparse_indices`` with ``sparse_block_size=1``. For TND input both take the
same cumulative ``actual_seq_lengths`` and the positions are batch-local.

``PrefillPlan`` validates and allocates both calls once; the attention plan
reads the indexer's index buffer in place, so ``run()`` is three kernel
launches on the current stream (score, top-k, attention) plus the SFA
token-list pass, with no host synchronisation between them.
"""
from __future__ import annotations

from .lightning_indexer import IndexerPlan
from .sparse_flash_attention import AttentionPlan


class PrefillPlan:
    def __init__(self, index_query, index_key, index_weights, query, key, query_rope, key_rope,
                 cu_seqlens, sparse_count=2048, scale_value=1.0, sparse_mode=3,
                 return_softmax_lse=False, return_value=False):
        self.indexer = IndexerPlan(index_query, index_key, index_weights, cu_seqlens, cu_seqlens,
                                   layout_query="TND", layout_key="TND", sparse_count=sparse_count,
                                   sparse_mode=sparse_mode, return_value=return_value)
        self.attention = AttentionPlan(query, key, key, self.indexer.idx, scale_value,
                                       actual_seq_lengths_query=cu_seqlens,
                                       actual_seq_lengths_kv=cu_seqlens, query_rope=query_rope,
                                       key_rope=key_rope, sparse_block_size=1, layout_query="TND",
                                       layout_kv="TND", sparse_mode=sparse_mode,
                                       return_softmax_lse=return_softmax_lse)
        if self.attention.si.data_ptr() != self.indexer.idx.data_ptr():
            raise RuntimeError("attention plan does not read the indexer's index buffer in place")

    @property
    def indices(self):
        return self.indexer.idx

    @property
    def values(self):
        return self.indexer.vals

    def run(self):
        """Returns (indices, attention_out, softmax_max, softmax_sum)."""
        self.indexer.run()
        out = self.attention.run()
        return (self.indexer.idx,) + tuple(out)


def dsa_prefill(index_query, index_key, index_weights, query, key, query_rope, key_rope, cu_seqlens,
                sparse_count=2048, scale_value=1.0, sparse_mode=3, return_softmax_lse=False):
    """One-shot form of ``PrefillPlan(...).run()``."""
    return PrefillPlan(index_query, index_key, index_weights, query, key, query_rope, key_rope,
                       cu_seqlens, sparse_count, scale_value, sparse_mode, return_softmax_lse).run()
