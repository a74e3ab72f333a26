"""``sparse_lightning_indexer_grad_kl_loss`` — drop-in for
``sparse_lightning_indexer_grad_kl_loss_triton``
(sparse_lightning_indexer_grad_kl_loss_triton.py:496-577) on MI355X.

The indexer's training signal: the KL divergence between the attention's mass on
each query row's selected tokens (teacher, from the SFA forward's softmax stats)
and the softmax of the indexer scores over the same tokens (student), with its
gradients for the indexer query, key and head weights. BSND only, sparse_mode 3,
N2 = Nidx2 = 1, as the reference. Returns ``(d_query_index, d_key_index,
d_weights, loss)`` with the inputs' dtypes and a float32 loss of shape (1,).
Semantics: sli_grad_kl_loss_numpy.py:17-180 with the row bounds of the
reference kernel (:63-69).
"""
from __future__ import annotations

import torch

from . import _host as H
from . import _lib

INT64_MAX = H.INT64_MAX


def _check_shapes(query, key, query_index, key_index, weights, sparse_indices, softmax_max, softmax_sum,
                  query_rope, key_rope):
    """Every tensor against query [B, S1, N1, D] and key [B, S2, 1, D]: the kernels index
    each one with B * S1 rows and S2 keys, so a mismatch would read outside it. Runs before
    any device check, so it needs no GPU."""
    for t, n in ((query, "query"), (key, "key"), (query_index, "query_index"), (key_index, "key_index")):
        if t.dim() != 4:
            raise ValueError(f"{n} must be a 4D BSND tensor, got {tuple(t.shape)}")
    B, S1, N1, D = query.shape
    S2 = key.shape[1]
    if key.shape[0] != B or key.shape[3] != D:
        raise ValueError(f"key must be [B={B}, S2, 1, D={D}], got {tuple(key.shape)}")
    if tuple(query_index.shape[:2]) != (B, S1):
        raise ValueError(f"query_index must be [B={B}, S1={S1}, Nidx1, D_idx], got {tuple(query_index.shape)}")
    Nidx1, Didx = query_index.shape[2], query_index.shape[3]
    if tuple(key_index.shape) != (B, S2, key_index.shape[2], Didx):
        raise ValueError(f"key_index must be [B={B}, S2={S2}, 1, D_idx={Didx}], got {tuple(key_index.shape)}")
    if tuple(weights.shape) != (B, S1, Nidx1):
        raise ValueError(f"weights must be [B={B}, S1={S1}, Nidx1={Nidx1}], got {tuple(weights.shape)}")
    if tuple(sparse_indices.shape[:3]) != (B, S1, 1):
        raise ValueError(f"sparse_indices must be [B={B}, S1={S1}, 1, topK], got {tuple(sparse_indices.shape)}")
    for t, n in ((softmax_max, "softmax_max"), (softmax_sum, "softmax_sum")):
        if t.numel() != B * S1 * N1 or (t.dim() == 4 and tuple(t.shape) != (B, 1, S1, N1)):
            raise ValueError(f"{n} must be [B={B}, 1, S1={S1}, N1={N1}], got {tuple(t.shape)}")
    if (query_rope is None) != (key_rope is None):
        raise ValueError("query_rope and key_rope must both be given or both be None")
    if query_rope is not None:
        Dr = query_rope.shape[-1]
        if query_rope.dim() != 4 or tuple(query_rope.shape[:3]) != (B, S1, N1):
            raise ValueError(f"query_rope must be [B={B}, S1={S1}, N1={N1}, Dr], got {tuple(query_rope.shape)}")
        if key_rope.dim() != 4 or tuple(key_rope.shape) != (B, S2, 1, Dr):
            raise ValueError(f"key_rope must be [B={B}, S2={S2}, 1, Dr={Dr}], got {tuple(key_rope.shape)}")


class KLLossPlan:
    """Validated arguments, outputs and workspace of one call; ``run()`` launches on
    the current stream."""

    def __init__(self, query, key, query_index, key_index, weights, sparse_indices, softmax_max,
                 softmax_sum, query_rope=None, key_rope=None, actual_seq_qlen=None,
                 actual_seq_klen=None, scale_value=1.0, layout="BSND", sparse_mode=3,
                 pre_tokens=INT64_MAX, next_tokens=INT64_MAX, deterministic=False):
        # validation: the reference's conditions (:510-514)
        if layout != "BSND":
            raise ValueError("Only BSND layout is supported in triton path")
        if sparse_mode != 3:
            raise ValueError("Only sparse_mode=3 (rightDownCausal) is supported")
        if sparse_indices.dim() != 4 or sparse_indices.shape[2] != 1:
            raise ValueError("Nidx2 must be 1 (MQA constraint)")
        _check_shapes(query, key, query_index, key_index, weights, sparse_indices, softmax_max,
                      softmax_sum, query_rope, key_rope)
        act_q = H.batch_lengths(actual_seq_qlen, query.shape[0], query.shape[1], "actual_seq_qlen")
        act_k = H.batch_lengths(actual_seq_klen, query.shape[0], key.shape[1], "actual_seq_klen")
        dev = H.require_device(query, key, query_index, key_index, weights, sparse_indices,
                               softmax_max, softmax_sum, query_rope, key_rope)
        lib = _lib.load()
        io = H.dtype_code(query.dtype, "query")
        for t, n in ((key, "key"), (query_index, "query_index"), (key_index, "key_index"),
                     (query_rope, "query_rope"), (key_rope, "key_rope")):
            if t is not None and t.dtype != query.dtype:
                raise ValueError(f"{n} dtype {t.dtype} differs from query dtype {query.dtype}")
        wdt = H.dtype_code(weights.dtype, "weights", allow_f32=True)
        B, S1, N1, D = query.shape
        S2, N2 = key.shape[1], key.shape[2]
        Nidx1, Didx = query_index.shape[2], query_index.shape[3]
        if N2 != 1 or key_index.shape[2] != 1:
            raise ValueError("Only N2=1 / Nidx2=1 (MQA) is supported")
        if (query_rope is None) != (key_rope is None):
            raise ValueError("query_rope and key_rope must both be given or both be None")
        Dr = 0 if query_rope is None else query_rope.shape[-1]
        topk = int(sparse_indices.shape[-1])
        self.q, self.k, self.qi, self.ki = (t.contiguous() for t in (query, key, query_index, key_index))
        self.qr = query_rope.contiguous() if query_rope is not None else None
        self.kr = key_rope.contiguous() if key_rope is not None else None
        self.w = weights.contiguous()
        self.si = sparse_indices.to(torch.int32).contiguous()
        self.sm_max = softmax_max.to(torch.float32).contiguous()
        self.sm_sum = softmax_sum.to(torch.float32).contiguous()
        self.dqi = torch.empty_like(self.qi)
        self.dki = torch.empty_like(self.ki)
        self.dw = torch.empty_like(self.w)
        self.loss = torch.empty(1, dtype=torch.float32, device=dev)
        self.ws_bytes = lib.dsa_sli_grad_workspace_bytes(B, S1, S2, topk, Didx)
        self.ws = torch.empty(max(self.ws_bytes, 1), dtype=torch.uint8, device=dev)
        self.d_aq, self.d_ak = H.i32(act_q, dev), H.i32(act_k, dev)
        self.lib, self.io, self.wdt, self.dev = lib, io, wdt, dev
        self.dims = (B, S1, S2, N1, D, Dr, Nidx1, Didx, topk)
        self.scale = float(scale_value)

    def run(self):
        B, S1, S2, N1, D, Dr, Nidx1, Didx, topk = self.dims
        _lib.check(self.lib.dsa_sli_grad_kl_loss(
            self.q.data_ptr(), self.k.data_ptr(), H.ptr(self.qr), H.ptr(self.kr), self.qi.data_ptr(),
            self.ki.data_ptr(), self.w.data_ptr(), self.io, self.wdt, self.si.data_ptr(), topk,
            self.sm_max.data_ptr(), self.sm_sum.data_ptr(), self.d_aq.data_ptr(), self.d_ak.data_ptr(),
            B, S1, S2, N1, D, Dr, Nidx1, Didx, self.scale, self.dqi.data_ptr(), self.dki.data_ptr(),
            self.dw.data_ptr(), self.loss.data_ptr(), self.ws.data_ptr(), self.ws_bytes,
            H.stream_ptr(self.dev)), "dsa_sli_grad_kl_loss")
        return self.dqi, self.dki, self.dw, self.loss


def sparse_lightning_indexer_grad_kl_loss(query, key, query_index, key_index, weights, sparse_indices,
                                          softmax_max, softmax_sum, query_rope=None, key_rope=None,
                                          actual_seq_qlen=None, actual_seq_klen=None, scale_value=1.0,
                                          layout="BSND", sparse_mode=3, pre_tokens=INT64_MAX,
                                          next_tokens=INT64_MAX, deterministic=False):
    """MI355X sparse lightning-indexer grad KL loss (arguments and returns as
    sparse_lightning_indexer_grad_kl_loss_triton.py:496-508)."""
    return KLLossPlan(query, key, query_index, key_index, weights, sparse_indices, softmax_max,
                      softmax_sum, query_rope, key_rope, actual_seq_qlen, actual_seq_klen, scale_value,
                      layout, sparse_mode, pre_tokens, next_tokens, deterministic).run()


class SparseLightningIndexerGradKLLoss(torch.nn.Module):
    """Module twin of ``SparseLightningIndexerGradKLLossTriton``
    (sparse_lightning_indexer_grad_kl_loss_triton.py:443-493)."""

    def __init__(self, scale_value=1.0, layout="BSND", sparse_mode=3, pre_tokens=INT64_MAX,
                 next_tokens=INT64_MAX, deterministic=False):
        super().__init__()
        self.scale_value, self.layout, self.sparse_mode = scale_value, layout, sparse_mode
        self.pre_tokens, self.next_tokens, self.deterministic = pre_tokens, next_tokens, deterministic

    def forward(self, query, key, query_index, key_index, weights, sparse_indices, softmax_max,
                softmax_sum, query_rope=None, key_rope=None, actual_seq_qlen=None, actual_seq_klen=None):
        return sparse_lightning_indexer_grad_kl_loss(
            query, key, query_index, key_index, weights, sparse_indices, softmax_max, softmax_sum,
            query_rope, key_rope, actual_seq_qlen, actual_seq_klen, self.scale_value, self.layout,
            self.sparse_mode, self.pre_tokens, self.next_tokens, self.deterministic)
