"""``sparse_flash_attention_grad`` — drop-in for ``sparse_flash_attention_grad_triton``
(sparse_flash_attention_grad_triton.py:498-677) on MI355X.

MLA-absorb, N2 = 1: ``value`` is ignored in the computation (key[..., :D] serves
as V) but its gradient ``d_value`` (the P^T dO path) is returned separately from
``d_key`` (the dS^T Q path), as in the reference; a caller whose key and value
share one tensor sums the two. Layouts BSND / TND; softmax stats (B,1,S1,N1) for
BSND and (1,T1,N1) for TND, as the forward returns them. Semantics are the
golden's (sparse_flash_attention_grad_numpy.py:34-143); TND is handled inside the
kernels through packed-row offsets instead of the reference's de-packing copies
(:562-578, :669-674).
"""
from __future__ import annotations

import ctypes

import torch

from . import _host as H
from . import _lib

INT64_MAX = H.INT64_MAX
VALID_D = (128, 256, 512)
D_ROPE = 64
VALID_N1 = (1, 2, 4, 8, 16, 32, 64, 128)


class GradPlan:
    """Validated arguments of one sparse_flash_attention_grad call (outputs, workspace,
    int32 index arrays); ``run()`` launches on the current stream."""

    def __init__(self, query, key, value, sparse_indices, d_out, out, softmax_max, softmax_sum,
                 scale_value=1.0, query_rope=None, key_rope=None, actual_seq_lengths_query=None,
                 actual_seq_lengths_kv=None, sparse_block_size=1, layout="BSND", sparse_mode=3,
                 pre_tokens=INT64_MAX, next_tokens=INT64_MAX, deterministic=False):
        # validation: same conditions and messages as the reference (:544-594)
        if pre_tokens != INT64_MAX or next_tokens != INT64_MAX:
            raise ValueError("pre_tokens/next_tokens only support default INT64_MAX")
        if sparse_mode not in (0, 3):
            raise ValueError("Only sparse_mode 0 (full) / 3 (rightDownCausal) supported")
        if query_rope is None or key_rope is None:
            raise ValueError("query_rope and key_rope are required (no empty rope)")
        if deterministic:
            raise ValueError("deterministic=True is not supported (scatter-add path)")
        if sparse_block_size < 1 or (sparse_block_size & (sparse_block_size - 1)) != 0 \
                or sparse_block_size > 128:
            raise ValueError("sparse_block_size must be a power of 2 in [1,128]")
        if layout not in ("BSND", "TND"):
            raise ValueError(f"unsupported layout {layout}")
        is_tnd = layout == "TND"
        dev = H.require_device(query, key, query_rope, key_rope, sparse_indices, d_out, out,
                               softmax_max, softmax_sum)
        lib = _lib.load()
        io = H.dtype_code(query.dtype, "query")
        for t, n in ((key, "key"), (query_rope, "query_rope"), (key_rope, "key_rope"),
                     (d_out, "d_out"), (out, "out")):
            if t.dtype != query.dtype:
                raise ValueError(f"{n} dtype {t.dtype} differs from query dtype {query.dtype}")

        if is_tnd:
            act_q = H.per_batch_from_cumsum(H.host_lengths(actual_seq_lengths_query))
            act_k = H.per_batch_from_cumsum(H.host_lengths(actual_seq_lengths_kv))
            B = len(act_q)
            T1, N1, D = query.shape
            n2 = key.shape[1]
            row_start = H.prefix(act_q)
            key_start = H.prefix(act_k)[:-1]
            if row_start[-1] > T1:
                raise ValueError("actual_seq_lengths_query exceeds the packed query length")
            if sum(act_k) > key.shape[0]:
                raise ValueError("actual_seq_lengths_kv exceeds the packed key length")
            total_rows = T1
            S2 = max(act_k) if act_k else 0
            sm_shape = (1, T1, N1)
        else:
            B, S1, N1, D = query.shape
            S2, n2 = key.shape[1], key.shape[2]
            act_q = H.host_lengths(actual_seq_lengths_query, B, S1)
            act_k = H.host_lengths(actual_seq_lengths_kv, key.shape[0], S2)
            row_start = [b * S1 for b in range(B + 1)]
            key_start = [b * S2 for b in range(key.shape[0])]
            total_rows = B * S1
            sm_shape = (B, 1, S1, N1)
        if len(act_k) != B:
            raise ValueError(f"batch mismatch: {B} query batches, {len(act_k)} kv lengths")
        Dr = query_rope.shape[-1]
        if D not in VALID_D:
            raise ValueError(f"D must be one of {VALID_D}, got {D}")
        if Dr != D_ROPE:
            raise ValueError(f"rope dim must be {D_ROPE}, got {Dr}")
        if n2 != 1:
            raise ValueError("Only N2=1 (MQA) is supported")
        if N1 not in VALID_N1:
            raise ValueError(f"N1 must be one of {VALID_N1}, got {N1}")
        if tuple(d_out.shape) != tuple(query.shape) or tuple(out.shape) != tuple(query.shape):
            raise ValueError("d_out and out must have the query's shape")
        if tuple(softmax_max.shape) != sm_shape or tuple(softmax_sum.shape) != sm_shape:
            raise ValueError(f"softmax_max / softmax_sum must have shape {sm_shape}")

        count = int(sparse_indices.shape[-1])
        si = sparse_indices.to(torch.int32).reshape(-1, count).contiguous()
        if si.shape[0] != total_rows:
            raise ValueError(f"sparse_indices rows {si.shape[0]} != query rows {total_rows}")
        self.q, self.qr = query.contiguous(), query_rope.contiguous()
        self.kk, self.kr = key.contiguous(), key_rope.contiguous()
        self.do, self.o = d_out.contiguous(), out.contiguous()
        self.sm_max = softmax_max.to(torch.float32).contiguous()
        self.sm_sum = softmax_sum.to(torch.float32).contiguous()
        self.si = si
        self.key_rows = self.kk.numel() // D
        if self.kr.numel() // Dr != self.key_rows:
            raise ValueError("key and key_rope hold different numbers of rows")

        self.dq = torch.empty_like(self.q)
        self.dqr = torch.empty_like(self.qr)
        self.dk = torch.empty_like(self.kk)
        self.dkr = torch.empty_like(self.kr)
        v_shape = tuple(value.shape) if value is not None else tuple(key.shape)
        if value is not None and value.numel() != self.kk.numel():
            raise ValueError("value must have the key's shape (MLA-absorb)")
        self.dv = torch.empty(v_shape, dtype=query.dtype, device=dev)

        self.lib, self.io, self.dev = lib, io, dev
        self.count, self.sbs = count, sparse_block_size
        self.B, self.total_rows, self.N1, self.D, self.Dr, self.S2 = B, total_rows, N1, D, Dr, S2
        self.sparse_mode, self.scale = sparse_mode, float(scale_value)
        # host copies of the row offsets and kv lengths size the per-batch dense buffers
        self.h_row_start = (ctypes.c_int32 * len(row_start))(*row_start)
        self.h_act_k = (ctypes.c_int32 * len(act_k))(*act_k)
        self.ws_bytes = lib.dsa_sfa_bwd_workspace_bytes(B, ctypes.cast(self.h_row_start, ctypes.c_void_p),
                                                        ctypes.cast(self.h_act_k, ctypes.c_void_p), S2,
                                                        total_rows, N1, D, count, sparse_block_size,
                                                        self.key_rows)
        if self.ws_bytes == 0:
            raise ValueError("dsa_sfa_bwd_workspace_bytes rejected the shapes")
        self.ws = torch.empty(max(self.ws_bytes, 1), dtype=torch.uint8, device=dev)
        self.d_row_start = H.i32(row_start, dev)
        self.d_key_start = H.i32(key_start if key_start else [0], dev)
        self.d_aq = H.i32(act_q, dev)
        self.d_ak = H.i32(act_k, dev)

    def run(self):
        _lib.check(self.lib.dsa_sfa_bwd(
            self.q.data_ptr(), self.qr.data_ptr(), self.kk.data_ptr(), self.kr.data_ptr(), self.io,
            self.si.data_ptr(), self.count, self.sbs, self.d_row_start.data_ptr(),
            self.d_key_start.data_ptr(), self.d_aq.data_ptr(), self.d_ak.data_ptr(),
            ctypes.cast(self.h_row_start, ctypes.c_void_p), ctypes.cast(self.h_act_k, ctypes.c_void_p), self.B,
            self.total_rows, self.N1, self.D, self.Dr, self.S2, self.key_rows, self.sparse_mode,
            self.scale, self.do.data_ptr(), self.o.data_ptr(), self.sm_max.data_ptr(),
            self.sm_sum.data_ptr(), self.dq.data_ptr(), self.dqr.data_ptr(), self.dk.data_ptr(),
            self.dkr.data_ptr(), self.dv.data_ptr(), self.ws.data_ptr(), self.ws_bytes,
            H.stream_ptr(self.dev)), "dsa_sfa_bwd")
        return self.dq, self.dk, self.dv, self.dqr, self.dkr


def sparse_flash_attention_grad(query, key, value, sparse_indices, d_out, out, softmax_max,
                                softmax_sum, scale_value=1.0, query_rope=None, key_rope=None,
                                actual_seq_lengths_query=None, actual_seq_lengths_kv=None,
                                sparse_block_size=1, layout="BSND", sparse_mode=3,
                                pre_tokens=INT64_MAX, next_tokens=INT64_MAX, deterministic=False):
    """MI355X sparse flash attention backward (arguments and returns as
    sparse_flash_attention_grad_triton.py:498-541): returns
    ``(d_query, d_key, d_value, d_query_rope, d_key_rope)``."""
    return GradPlan(query, key, value, sparse_indices, d_out, out, softmax_max, softmax_sum,
                    scale_value, query_rope, key_rope, actual_seq_lengths_query,
                    actual_seq_lengths_kv, sparse_block_size, layout, sparse_mode, pre_tokens,
                    next_tokens, deterministic).run()


class SparseFlashAttentionGrad(torch.nn.Module):
    """Module twin of ``SparseFlashAttentionGradTriton`` (sparse_flash_attention_grad_triton.py:680-721)."""

    def __init__(self, scale_value=1.0, sparse_block_size=1, layout="BSND", sparse_mode=3,
                 pre_tokens=INT64_MAX, next_tokens=INT64_MAX, deterministic=False):
        super().__init__()
        self.scale_value = scale_value
        self.sparse_block_size = sparse_block_size
        self.layout = layout
        self.sparse_mode = sparse_mode
        self.pre_tokens = pre_tokens
        self.next_tokens = next_tokens
        self.deterministic = deterministic

    def forward(self, query, key, value, sparse_indices, d_out, out, softmax_max, softmax_sum,
                query_rope=None, key_rope=None, actual_seq_lengths_query=None,
                actual_seq_lengths_kv=None):
        return sparse_flash_attention_grad(
            query, key, value, sparse_indices, d_out, out, softmax_max, softmax_sum,
            scale_value=self.scale_value, query_rope=query_rope, key_rope=key_rope,
            actual_seq_lengths_query=actual_seq_lengths_query,
            actual_seq_lengths_kv=actual_seq_lengths_kv, sparse_block_size=self.sparse_block_size,
            layout=self.layout, sparse_mode=self.sparse_mode, pre_tokens=self.pre_tokens,
            next_tokens=self.next_tokens, deterministic=self.deterministic)
