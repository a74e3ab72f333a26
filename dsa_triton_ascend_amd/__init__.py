"""MI355X-native DeepSeek Sparse Attention hot path.

Drop-in operators with the reference's Python signatures:

* :func:`lightning_indexer` (lightning_indexer_triton.py:466) — indexer score + stable top-k
* :func:`sparse_flash_attention` (sparse_flash_attention_triton.py:1295) — MLA-absorb SFA forward
* :func:`sparse_flash_attention_grad` (sparse_flash_attention_grad_triton.py:498) — its backward
* :func:`sparse_lightning_indexer_grad_kl_loss` (sparse_lightning_indexer_grad_kl_loss_triton.py:496)
  — the indexer's KL training loss and its gradients

and :class:`PrefillPlan` / :func:`dsa_prefill`, the two chained on one packed
(TND) batch with the indexer's top-k feeding the attention in place.

Both run hand-written gfx950 HIP kernels through the C ABI of
``libdsa_mi355x.so`` (include/dsa_mi355x.h); PyTorch tensors are only buffers.
"""
from .lightning_indexer import LightningIndexer, lightning_indexer
from .pipeline import PrefillPlan, dsa_prefill
from .sparse_flash_attention import SparseFlashAttention, sparse_flash_attention
from .sparse_flash_attention_grad import SparseFlashAttentionGrad, sparse_flash_attention_grad
from .sli_grad_kl_loss import SparseLightningIndexerGradKLLoss, sparse_lightning_indexer_grad_kl_loss
from .dense_loss import (DenseLightningIndexerGradKLLoss, DenseLightningIndexerSoftmaxLse, DenseLossBackward,
                         dense_lightning_indexer_grad_kl_loss, dense_lightning_indexer_softmax_lse,
                         dense_loss_backward, npu_dense_lightning_indexer_grad_kl_loss,
                         npu_dense_lightning_indexer_softmax_lse)

__all__ = ["lightning_indexer", "LightningIndexer", "sparse_flash_attention", "SparseFlashAttention",
           "sparse_flash_attention_grad", "SparseFlashAttentionGrad", "sparse_lightning_indexer_grad_kl_loss",
           "SparseLightningIndexerGradKLLoss", "dense_lightning_indexer_softmax_lse",
           "npu_dense_lightning_indexer_softmax_lse", "dense_loss_backward",
           "dense_lightning_indexer_grad_kl_loss", "npu_dense_lightning_indexer_grad_kl_loss",
           "DenseLightningIndexerSoftmaxLse", "DenseLossBackward", "DenseLightningIndexerGradKLLoss",
           "PrefillPlan", "dsa_prefill"]
