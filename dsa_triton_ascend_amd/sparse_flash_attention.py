"""``sparse_flash_attention`` — drop-in for ``sparse_flash_attention_triton``
(sparse_flash_attention_triton.py:1295-1455) on MI355X.

MLA-absorb (attention_mode 2), N2 = 1: the ``value`` argument is ignored and
key[..., :D] serves as V. Layouts BSND / TND for the query and BSND / TND /
PA_BSND for the KV; outputs ``(attention_out q-dtype, softmax_max,
softmax_sum)`` with the stats shaped (B,1,S1,N1) for BSND queries and
(1,T1,N1) for TND (zeros when ``return_softmax_lse`` is False).
Semantics are the golden's (sparse_flash_attention_numpy.py:38-160).

TND and PA_BSND are handled inside the kernels (packed-row offsets and a
block-table lookup per gathered token) instead of the reference's host-side
de-packing / de-paging copies (:975-1033).
"""
from __future__ import annotations

import torch

from . import _host as H
from . import _lib

INT64_MAX = H.INT64_MAX
VALID_D = (128, 256, 512)
D_ROPE = 64
VALID_N1 = (1, 2, 4, 8, 16, 32, 64, 128)


class AttentionPlan:
    """Validated arguments of one sparse_flash_attention call (outputs,
    workspace, int32 index arrays); ``run()`` launches on the current stream."""

    def __init__(self, query, key, value, sparse_indices, scale_value=1.0, block_table=None,
                 actual_seq_lengths_query=None, actual_seq_lengths_kv=None,
                 query_rope=None, key_rope=None, sparse_block_size=1,
                 layout_query="BSND", layout_kv="BSND", sparse_mode=0,
                 pre_tokens=INT64_MAX, next_tokens=INT64_MAX, attention_mode=2,
                 return_softmax_lse=False, block_size=0, kv_splits=0):
        # validation: same conditions and messages as the reference (:1341-1351)
        if attention_mode != 2:
            raise ValueError("Only attention_mode=2 (MLA-absorb) is supported")
        if pre_tokens != INT64_MAX or next_tokens != INT64_MAX:
            raise ValueError("pre_tokens/next_tokens only support default INT64_MAX")
        if sparse_mode not in (0, 3):
            raise ValueError("Only sparse_mode 0 (full) / 3 (rightDownCausal) supported")
        if query_rope is None or key_rope is None:
            raise ValueError("query_rope and key_rope are required (no empty rope)")
        if sparse_block_size < 1 or (sparse_block_size & (sparse_block_size - 1)) != 0 \
                or sparse_block_size > 128:
            raise ValueError("sparse_block_size must be a power of 2 in [1,128]")
        if layout_query not in ("BSND", "TND") or layout_kv not in ("BSND", "TND", "PA_BSND"):
            raise ValueError(f"unsupported layout {layout_query}/{layout_kv}")
        is_tnd_q = layout_query == "TND"
        is_tnd_kv = layout_kv == "TND"
        is_pa = layout_kv == "PA_BSND"
        if is_pa and block_table is None:
            raise ValueError("PA_BSND requires block_table")
        dev = H.require_device(query, key, query_rope, key_rope, sparse_indices,
                               block_table if is_pa else None)
        lib = _lib.load()
        io = H.dtype_code(query.dtype, "query")
        for t, n in ((key, "key"), (query_rope, "query_rope"), (key_rope, "key_rope")):
            if t.dtype != query.dtype:
                raise ValueError(f"{n} dtype {t.dtype} differs from query dtype {query.dtype}")

        # ---- query side
        if is_tnd_q:
            act_q = H.per_batch_from_cumsum(H.host_lengths(actual_seq_lengths_query))
            B = len(act_q)
            T1, N1, D = query.shape
            row_start = H.prefix(act_q)
            if row_start[-1] > T1:
                raise ValueError("actual_seq_lengths_query exceeds the packed query length")
            total_rows = T1
        else:
            B, S1, N1, D = query.shape
            act_q = H.host_lengths(actual_seq_lengths_query, B, S1)
            row_start = [b * S1 for b in range(B + 1)]
            total_rows = B * S1
        Dr = query_rope.shape[-1]

        # ---- kv side
        d_bt = None
        max_blocks = page_bs = 0
        if is_tnd_kv:
            act_k = H.per_batch_from_cumsum(H.host_lengths(actual_seq_lengths_kv))
            key_start = H.prefix(act_k)[:-1]
            S2 = max(act_k) if act_k else 0
            n2 = key.shape[1]
        elif is_pa:
            act_k = H.host_lengths(actual_seq_lengths_kv)
            page_bs = int(block_size or key.shape[1])
            max_blocks = int(block_table.shape[1])
            S2 = max_blocks * page_bs
            key_start = [0] * B
            n2 = key.shape[2]
            d_bt = block_table.to(torch.int32).contiguous()
        else:
            S2 = key.shape[1]
            n2 = key.shape[2]
            act_k = H.host_lengths(actual_seq_lengths_kv, key.shape[0], S2)
            key_start = [b * S2 for b in range(key.shape[0])]
        if is_tnd_kv and sum(act_k) > key.shape[0]:
            raise ValueError("actual_seq_lengths_kv exceeds the packed key length")
        if len(act_k) != B:
            raise ValueError(f"batch mismatch: {B} query batches, {len(act_k)} kv lengths")

        # ---- shape checks (:1391-1398)
        if D not in VALID_D:
            raise ValueError(f"D must be one of {VALID_D}, got {D}")
        if Dr != D_ROPE:
            raise ValueError(f"rope dim must be {D_ROPE}, got {Dr}")
        if n2 != 1:
            raise ValueError("Only N2=1 (MQA) is supported")
        if N1 not in VALID_N1:
            raise ValueError(f"N1 must be one of {VALID_N1}, got {N1}")

        count = int(sparse_indices.shape[-1])
        si = sparse_indices.to(torch.int32).reshape(-1, count).contiguous()
        if si.shape[0] != total_rows:
            raise ValueError(f"sparse_indices rows {si.shape[0]} != query rows {total_rows}")
        q = query.contiguous()
        qr = query_rope.contiguous()
        kk = key.contiguous()
        kr = key_rope.contiguous()

        out_shape = (T1, N1, D) if is_tnd_q else (B, S1, N1, D)
        out = torch.empty(out_shape, dtype=query.dtype, device=dev)
        sm_shape = (1, T1, N1) if is_tnd_q else (B, 1, S1, N1)
        if return_softmax_lse:
            sm_max = torch.empty(sm_shape, dtype=torch.float32, device=dev)
            sm_sum = torch.empty(sm_shape, dtype=torch.float32, device=dev)
        else:
            sm_max = sm_sum = None
        self.lib, self.io, self.dev = lib, io, dev
        self.q, self.qr, self.kk, self.kr, self.si = q, qr, kk, kr, si
        self.out, self.sm_max, self.sm_sum, self.sm_shape = out, sm_max, sm_sum, sm_shape
        self.return_lse = return_softmax_lse
        self.count, self.sbs, self.d_bt, self.max_blocks, self.page_bs = count, sparse_block_size, d_bt, max_blocks, page_bs
        self.B, self.total_rows, self.N1, self.D, self.Dr, self.S2 = B, total_rows, N1, D, Dr, S2
        self.sparse_mode, self.scale, self.kv_splits = sparse_mode, float(scale_value), int(kv_splits)
        self.ws_bytes = lib.dsa_sfa_workspace_bytes(total_rows, N1, D, count, sparse_block_size,
                                                    int(kv_splits)) if total_rows > 0 else 0
        # the workspace starts with a zero KV row that the library keeps at zero across
        # calls; only that prefix needs clearing (include/dsa_mi355x.h, dsa_sfa_fwd)
        self.ws = torch.empty(max(self.ws_bytes, 1), dtype=torch.uint8, device=dev)
        self.ws[:min(self.ws.numel(), lib.dsa_sfa_workspace_zero_bytes())].zero_()
        self.d_row_start = H.i32(row_start, dev)
        self.d_key_start = H.i32(key_start, dev)
        self.d_aq = H.i32(act_q, dev)
        self.d_ak = H.i32(act_k, dev)
        self.act_q, self.act_k, self.row_start = act_q, act_k, row_start
        self.key_rows = kk.numel() // D

    def run(self):
        if self.total_rows > 0:
            _lib.check(self.lib.dsa_sfa_fwd(
                self.q.data_ptr(), self.qr.data_ptr(), self.kk.data_ptr(), self.kr.data_ptr(),
                self.io, self.si.data_ptr(), self.count, self.sbs, H.ptr(self.d_bt),
                self.max_blocks, self.page_bs, self.d_row_start.data_ptr(),
                self.d_key_start.data_ptr(), self.d_aq.data_ptr(), self.d_ak.data_ptr(), self.B,
                self.total_rows, self.N1, self.D, self.Dr, self.S2, self.key_rows, self.sparse_mode,
                self.scale,
                self.out.data_ptr(), H.ptr(self.sm_max), H.ptr(self.sm_sum), self.ws.data_ptr(),
                self.ws_bytes, self.kv_splits, H.stream_ptr(self.dev)), "dsa_sfa_fwd")
        if not self.return_lse:
            z = torch.zeros(self.sm_shape, dtype=torch.float32, device=self.dev)
            return self.out, z, z.clone()
        return self.out, self.sm_max, self.sm_sum


def sparse_flash_attention(query, key, value, sparse_indices, scale_value=1.0, block_table=None,
                           actual_seq_lengths_query=None, actual_seq_lengths_kv=None,
                           query_rope=None, key_rope=None, sparse_block_size=1,
                           layout_query="BSND", layout_kv="BSND", sparse_mode=0,
                           pre_tokens=INT64_MAX, next_tokens=INT64_MAX, attention_mode=2,
                           return_softmax_lse=False, block_size=0, kv_splits=0):
    """MI355X sparse flash attention forward (arguments as
    sparse_flash_attention_triton.py:1295-1338; ``kv_splits`` is an optional
    tuning knob for split-KV decode, 0 = library choice)."""
    return AttentionPlan(query, key, value, sparse_indices, scale_value, block_table,
                         actual_seq_lengths_query, actual_seq_lengths_kv, query_rope, key_rope,
                         sparse_block_size, layout_query, layout_kv, sparse_mode, pre_tokens,
                         next_tokens, attention_mode, return_softmax_lse, block_size,
                         kv_splits).run()


class SparseFlashAttention(torch.nn.Module):
    """Module twin of ``SparseFlashAttentionTriton`` (sparse_flash_attention_triton.py:1458-1509).
    Like the reference Cell, ``block_size`` is stored but not forwarded (:1508)."""

    def __init__(self, scale_value=1.0, sparse_block_size=1, layout_query="BSND", layout_kv="BSND",
                 sparse_mode=0, attention_mode=2, return_softmax_lse=False, pre_tokens=INT64_MAX,
                 next_tokens=INT64_MAX, block_size=0):
        super().__init__()
        self.scale_value = scale_value
        self.sparse_block_size = sparse_block_size
        self.layout_query = layout_query
        self.layout_kv = layout_kv
        self.sparse_mode = sparse_mode
        self.attention_mode = attention_mode
        self.return_softmax_lse = return_softmax_lse
        self.pre_tokens = pre_tokens
        self.next_tokens = next_tokens
        self.block_size = block_size

    def forward(self, query, key, value, sparse_indices, query_rope=None, key_rope=None,
                actual_seq_lengths_query=None, actual_seq_lengths_kv=None, block_table=None):
        return sparse_flash_attention(
            query, key, value, sparse_indices, scale_value=self.scale_value,
            block_table=block_table, actual_seq_lengths_query=actual_seq_lengths_query,
            actual_seq_lengths_kv=actual_seq_lengths_kv, query_rope=query_rope, key_rope=key_rope,
            sparse_block_size=self.sparse_block_size, layout_query=self.layout_query,
            layout_kv=self.layout_kv, sparse_mode=self.sparse_mode, pre_tokens=self.pre_tokens,
            next_tokens=self.next_tokens, attention_mode=self.attention_mode,
            return_softmax_lse=self.return_softmax_lse)
