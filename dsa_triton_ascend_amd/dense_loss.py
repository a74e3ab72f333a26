"""Dense lightning-indexer loss on MI355X — drop-ins for dense_loss_backward_triton.py:

* ``dense_lightning_indexer_softmax_lse`` (+ the ``npu_`` alias) <-
  ``npu_dense_lightning_indexer_softmax_lse_triton`` (:776-806): per query row the
  max and the sum of ``exp(I - max)`` of the indexer scores over the visible keys,
  shapes (B, 1, S1) float32;
* ``dense_loss_backward`` <- ``dense_loss_backward_triton`` (:709-774), and the
  ``dense_lightning_indexer_grad_kl_loss`` / ``npu_`` aliases (:828-890): the sparse
  KL loss with every visible key ``t < min(max(act_k - act_q + s1 + 1, 0), S2)`` as a
  slot, the teacher over grouped key heads (key [B, S2, N2, D], stats [B, N2, S1, G])
  and the indexer softmax normalised by the given stats (computed in the kernel when
  omitted). Returns ``(d_query_index, d_key_index, d_weights, loss)``.

BSND, sparse_mode 3 only, as the reference; its input checks and messages
(:605-706) are kept.
"""
from __future__ import annotations

import torch

from . import _host as H
from . import _lib

INT64_MAX = H.INT64_MAX
SUPPORTED_D = (128, 256, 512)
SUPPORTED_NIDX1 = (32, 64, 128)


def _check_in(name, value, supported):
    if value not in supported:
        raise ValueError(f"{name}={value} is not supported; expected one of {supported}")


def _validate_index(query_index, key_index, weights, layout, sparse_mode, pre_tokens, next_tokens):
    if layout != "BSND":
        raise ValueError("Only BSND layout is supported")
    if sparse_mode != 3:
        raise ValueError("Only sparse_mode=3 (rightDownCausal) is supported")
    if pre_tokens != INT64_MAX or next_tokens != INT64_MAX:
        raise ValueError("pre_tokens/next_tokens only support the official default value")
    if query_index.dim() != 4 or key_index.dim() != 4:
        raise ValueError("query_index and key_index must be 4D BSND tensors")
    if weights.dim() != 3:
        raise ValueError("weights must be [B, S1, Nidx1]")
    B, S1, Nidx1, D_idx = query_index.shape
    if key_index.shape[0] != B or key_index.shape[2] != 1:
        raise ValueError("key_index must be [B, S2, 1, D_idx]")
    if tuple(weights.shape) != (B, S1, Nidx1):
        raise ValueError("weights must be [B, S1, Nidx1]")
    if key_index.shape[3] != D_idx:
        raise ValueError("query_index and key_index must share D_idx")
    _check_in("Nidx1", Nidx1, SUPPORTED_NIDX1)
    _check_in("D_idx", D_idx, SUPPORTED_D)


def _reshape_stat(stat, B, S1, name):
    if tuple(stat.shape) in ((B, S1), (B * S1,), (B, 1, S1), (B, 1, S1, 1)):
        return stat.reshape(B * S1).contiguous()
    raise ValueError(f"{name} must have shape [B,S1], [B*S1], [B,1,S1], or [B,1,S1,1], got {tuple(stat.shape)}")


def dense_lightning_indexer_softmax_lse(query_index, key_index, weights, actual_seq_qlen=None,
                                        actual_seq_klen=None, layout="BSND", sparse_mode=3,
                                        pre_tokens=INT64_MAX, next_tokens=INT64_MAX):
    """Returns ``(softmax_max_index, softmax_sum_index)``, each (B, 1, S1) float32
    (dense_loss_backward_triton.py:776-806); rows without a visible key hold (-inf, 0)."""
    _validate_index(query_index, key_index, weights, layout, sparse_mode, pre_tokens, next_tokens)
    aq = H.batch_lengths(actual_seq_qlen, query_index.shape[0], query_index.shape[1], "actual_seq_qlen")
    ak = H.batch_lengths(actual_seq_klen, query_index.shape[0], key_index.shape[1], "actual_seq_klen")
    dev = H.require_device(query_index, key_index, weights)
    lib = _lib.load()
    io = H.dtype_code(query_index.dtype, "query_index")
    if key_index.dtype != query_index.dtype:
        raise TypeError("query_index and key_index must share dtype")
    wdt = H.dtype_code(weights.dtype, "weights", allow_f32=True)
    B, S1, Nidx1, Didx = query_index.shape
    S2 = key_index.shape[1]
    act_q, act_k = H.i32(aq, dev), H.i32(ak, dev)
    qi, ki, w = query_index.contiguous(), key_index.contiguous(), weights.contiguous()
    mx = torch.empty((B, 1, S1), dtype=torch.float32, device=dev)
    sm = torch.empty((B, 1, S1), dtype=torch.float32, device=dev)
    _lib.check(lib.dsa_dense_li_softmax_lse(qi.data_ptr(), ki.data_ptr(), w.data_ptr(), io, wdt,
                                            act_q.data_ptr(), act_k.data_ptr(), B, S1, S2, Nidx1, Didx,
                                            mx.data_ptr(), sm.data_ptr(), H.stream_ptr(dev)),
               "dsa_dense_li_softmax_lse")
    return mx, sm


npu_dense_lightning_indexer_softmax_lse = dense_lightning_indexer_softmax_lse


class DenseLossPlan:
    """Validated arguments, outputs and workspace of one dense loss call; ``run()``
    launches on the current stream."""

    def __init__(self, query, key, query_index, key_index, weights, softmax_max, softmax_sum,
                 softmax_max_index=None, softmax_sum_index=None, scale_value=1.0, query_rope=None,
                 key_rope=None, actual_seq_qlen=None, actual_seq_klen=None, layout="BSND",
                 sparse_mode=3, pre_tokens=INT64_MAX, next_tokens=INT64_MAX):
        # the reference's checks (:667-706)
        if query.dim() != 4 or key.dim() != 4:
            raise ValueError("query and key must be 4D BSND tensors")
        _validate_index(query_index, key_index, weights, layout, sparse_mode, pre_tokens, next_tokens)
        B, S1, N1, D = query.shape
        if key.shape[0] != B or key.shape[3] != D:
            raise ValueError("key must be [B, S2, N2, D_attn]")
        N2 = key.shape[2]
        if N2 <= 0 or N1 % N2 != 0:
            raise ValueError("query N1 must be divisible by key N2")
        if query_index.shape[0] != B or query_index.shape[1] != S1:
            raise ValueError("query_index must share B and S1 with query")
        if key_index.shape[1] != key.shape[1]:
            raise ValueError("key_index S2 must match key S2")
        sm_shape = (B, N2, S1, N1 // N2)
        if tuple(softmax_max.shape) != sm_shape or tuple(softmax_sum.shape) != sm_shape:
            raise ValueError(f"softmax_max and softmax_sum must be [B, N2, S1, G], got {tuple(softmax_max.shape)}")
        _check_in("D_attn", D, SUPPORTED_D)
        if (query_rope is None) != (key_rope is None):
            raise ValueError("query_rope and key_rope must be both provided or both omitted")
        Dr = 0
        if query_rope is not None:
            if query_rope.dim() != 4 or key_rope.dim() != 4:
                raise ValueError("query_rope and key_rope must be 4D BSND tensors")
            if tuple(query_rope.shape[:3]) != tuple(query.shape[:3]):
                raise ValueError("query_rope must share [B, S1, N1] with query")
            if tuple(key_rope.shape[:3]) != tuple(key.shape[:3]):
                raise ValueError("key_rope must share [B, S2, N2] with key")
            if query_rope.shape[3] != key_rope.shape[3]:
                raise ValueError("query_rope and key_rope must share Drope")
            if query_rope.shape[3] != 64:
                raise ValueError("Only Drope=64 is supported for query_rope/key_rope")
            if query_rope.dtype != query.dtype or key_rope.dtype != key.dtype:
                raise TypeError("query_rope/key_rope dtype must match query/key dtype")
            Dr = 64
        if query.dtype not in (torch.float16, torch.bfloat16):
            raise TypeError(f"query dtype must be float16 or bfloat16, got {query.dtype}")
        if key.dtype != query.dtype or query_index.dtype != query.dtype or key_index.dtype != query.dtype:
            raise TypeError("query, key, query_index, and key_index must share dtype")
        if weights.dtype != query.dtype and weights.dtype != torch.float32:
            raise TypeError("weights dtype must match query dtype or be float32")
        if softmax_max.dtype != torch.float32 or softmax_sum.dtype != torch.float32:
            raise TypeError("softmax_max and softmax_sum must be float32")
        if (softmax_max_index is None) != (softmax_sum_index is None):
            raise ValueError("softmax_max_index and softmax_sum_index must be both provided or both omitted")
        self.imax = self.isum = None
        if softmax_max_index is not None:
            if softmax_max_index.dtype != torch.float32 or softmax_sum_index.dtype != torch.float32:
                raise TypeError("softmax_max_index and softmax_sum_index must be float32")
            self.imax = _reshape_stat(softmax_max_index, B, S1, "softmax_max_index")
            self.isum = _reshape_stat(softmax_sum_index, B, S1, "softmax_sum_index")
        aq = H.batch_lengths(actual_seq_qlen, B, S1, "actual_seq_qlen")
        ak = H.batch_lengths(actual_seq_klen, B, key.shape[1], "actual_seq_klen")
        dev = H.require_device(query, key, query_index, key_index, weights, softmax_max, softmax_sum,
                               query_rope, key_rope, softmax_max_index, softmax_sum_index)
        lib = _lib.load()
        S2, Nidx1, Didx = key.shape[1], query_index.shape[2], query_index.shape[3]
        self.q, self.k, self.qi, self.ki = (t.contiguous() for t in (query, key, query_index, key_index))
        self.qr = query_rope.contiguous() if query_rope is not None else None
        self.kr = key_rope.contiguous() if key_rope is not None else None
        self.w = weights.contiguous()
        self.sm_max, self.sm_sum = softmax_max.contiguous(), softmax_sum.contiguous()
        self.dqi = torch.empty_like(self.qi)
        self.dki = torch.empty_like(self.ki)
        self.dw = torch.empty_like(self.w)
        self.loss = torch.empty(1, dtype=torch.float32, device=dev)
        self.ws_bytes = lib.dsa_dense_li_grad_workspace_bytes(B, S1, S2, Didx)
        self.ws = torch.empty(max(self.ws_bytes, 1), dtype=torch.uint8, device=dev)
        self.d_aq, self.d_ak = H.i32(aq, dev), H.i32(ak, dev)
        self.lib, self.dev = lib, dev
        self.io = H.dtype_code(query.dtype, "query")
        self.wdt = H.dtype_code(weights.dtype, "weights", allow_f32=True)
        self.dims = (B, S1, S2, N1, N2, D, Dr, Nidx1, Didx)
        self.scale = float(scale_value)

    def run(self):
        B, S1, S2, N1, N2, D, Dr, Nidx1, Didx = self.dims
        _lib.check(self.lib.dsa_dense_li_grad_kl_loss(
            self.q.data_ptr(), self.k.data_ptr(), H.ptr(self.qr), H.ptr(self.kr), self.qi.data_ptr(),
            self.ki.data_ptr(), self.w.data_ptr(), self.io, self.wdt, self.sm_max.data_ptr(),
            self.sm_sum.data_ptr(), H.ptr(self.imax), H.ptr(self.isum), self.d_aq.data_ptr(),
            self.d_ak.data_ptr(), B, S1, S2, N1, N2, D, Dr, Nidx1, Didx, self.scale, self.dqi.data_ptr(),
            self.dki.data_ptr(), self.dw.data_ptr(), self.loss.data_ptr(), self.ws.data_ptr(), self.ws_bytes,
            H.stream_ptr(self.dev)), "dsa_dense_li_grad_kl_loss")
        return self.dqi, self.dki, self.dw, self.loss


def dense_loss_backward(query, key, query_index, key_index, weights, softmax_max, softmax_sum,
                        softmax_max_index=None, softmax_sum_index=None, scale_value=1.0, query_rope=None,
                        key_rope=None, actual_seq_qlen=None, actual_seq_klen=None, layout="BSND",
                        sparse_mode=3, pre_tokens=INT64_MAX, next_tokens=INT64_MAX):
    """MI355X dense lightning-indexer KL loss backward (arguments and returns as
    dense_loss_backward_triton.py:709-774)."""
    return DenseLossPlan(query, key, query_index, key_index, weights, softmax_max, softmax_sum,
                         softmax_max_index, softmax_sum_index, scale_value, query_rope, key_rope,
                         actual_seq_qlen, actual_seq_klen, layout, sparse_mode, pre_tokens, next_tokens).run()


def dense_lightning_indexer_grad_kl_loss(query, key, query_index, key_index, weights, softmax_max,
                                         softmax_sum, softmax_max_index, softmax_sum_index, scale_value,
                                         query_rope=None, key_rope=None, actual_seq_qlen=None,
                                         actual_seq_klen=None, layout="BSND", sparse_mode=3,
                                         pre_tokens=INT64_MAX, next_tokens=INT64_MAX):
    """Official-style wrapper with the index stats required (dense_loss_backward_triton.py:828-860)."""
    return dense_loss_backward(query, key, query_index, key_index, weights, softmax_max, softmax_sum,
                               softmax_max_index, softmax_sum_index, scale_value, query_rope, key_rope,
                               actual_seq_qlen, actual_seq_klen, layout, sparse_mode, pre_tokens, next_tokens)


npu_dense_lightning_indexer_grad_kl_loss = dense_lightning_indexer_grad_kl_loss


class DenseLightningIndexerSoftmaxLse(torch.nn.Module):
    """Module twin of ``DenseLightningIndexerSoftmaxLseTriton`` (dense_loss_backward_triton.py:889-905)."""

    def forward(self, query_index, key_index, weight, actual_seq_qlen=None, actual_seq_klen=None,
                layout="BSND", sparse_mode=3, pre_tokens=INT64_MAX, next_tokens=INT64_MAX):
        return dense_lightning_indexer_softmax_lse(query_index, key_index, weight, actual_seq_qlen,
                                                   actual_seq_klen, layout, sparse_mode, pre_tokens, next_tokens)


class DenseLossBackward(torch.nn.Module):
    """Module twin of ``DenseLossBackwardTriton`` (dense_loss_backward_triton.py:908-937); a
    ``scale_value`` given to ``forward`` overrides the constructor's."""

    def __init__(self, scale_value=1.0, layout="BSND", sparse_mode=3, pre_tokens=INT64_MAX,
                 next_tokens=INT64_MAX):
        super().__init__()
        self.scale_value, self.layout, self.sparse_mode = scale_value, layout, sparse_mode
        self.pre_tokens, self.next_tokens = pre_tokens, next_tokens

    def forward(self, query, key, query_index, key_index, weights, softmax_max, softmax_sum,
                softmax_max_index=None, softmax_sum_index=None, scale_value=None, query_rope=None,
                key_rope=None, actual_seq_qlen=None, actual_seq_klen=None):
        scale = self.scale_value if scale_value is None else scale_value
        return dense_loss_backward(query, key, query_index, key_index, weights, softmax_max, softmax_sum,
                                   softmax_max_index, softmax_sum_index, scale, query_rope, key_rope,
                                   actual_seq_qlen, actual_seq_klen, self.layout, self.sparse_mode,
                                   self.pre_tokens, self.next_tokens)


class DenseLightningIndexerGradKLLoss(torch.nn.Module):
    """Module twin of ``DenseLightningIndexerGradKLLossTriton`` (dense_loss_backward_triton.py:940-960)."""

    def forward(self, query, key, query_index, key_index, weights, softmax_max, softmax_sum,
                softmax_max_index, softmax_sum_index, scale_value=1.0, query_rope=None, key_rope=None,
                actual_seq_qlen=None, actual_seq_klen=None, layout="BSND", sparse_mode=3,
                pre_tokens=INT64_MAX, next_tokens=INT64_MAX):
        return dense_lightning_indexer_grad_kl_loss(query, key, query_index, key_index, weights, softmax_max,
                                                    softmax_sum, softmax_max_index, softmax_sum_index,
                                                    scale_value, query_rope, key_rope, actual_seq_qlen,
                                                    actual_seq_klen, layout, sparse_mode, pre_tokens, next_tokens)
