"""``lightning_indexer`` — drop-in for ``lightning_indexer_triton``
(lightning_indexer_triton.py:466-554) on MI355X.

Same arguments, defaults, layouts (BSND / TND) and outputs
``(sparse_indices int32 [B,S1,N2,k] | [T1,N2,k], sparse_values q-dtype)``.
Ordering follows the numpy golden (lightning_indexer_numpy.py:92-105): scores
are quantised to the query dtype, then ordered by score descending with ties
broken by ascending key index; slots past the visible keys get index -1 and
value 0.

The device work is two C-ABI calls (``dsa_li_score`` then ``dsa_li_topk``); the
TND path indexes the packed tensors directly instead of padding them to BSND
(the reference's ``_tnd_to_bsnd`` / ``_bsnd_to_tnd``, :299-340).
"""
from __future__ import annotations

import torch

from . import _host as H
from . import _lib

INT64_MAX = H.INT64_MAX


def _score_ld(s2: int) -> int:
    return max(64, (s2 + 63) // 64 * 64)


class IndexerPlan:
    """Validated arguments of one lightning_indexer call: output buffers, the
    int32 index arrays the C ABI takes and the score scratch. ``score()`` and
    ``topk()`` launch the two kernels on the current stream (the bench times
    them separately); ``run()`` does both."""

    def __init__(self, query, key, weights, actual_seq_lengths_query=None,
                 actual_seq_lengths_key=None, block_table=None, layout_query="BSND",
                 layout_key="BSND", sparse_count=2048, sparse_mode=3, return_value=False):
        is_pa = layout_key == "PA_BSND"
        if block_table is not None and not is_pa:
            raise ValueError("PA_BSND / block_table not supported in triton lightning_indexer")
        if is_pa and block_table is None:
            raise ValueError("PA_BSND requires block_table")
        if layout_query not in ("BSND", "TND") or layout_key not in ("BSND", "TND", "PA_BSND"):
            raise ValueError(f"unsupported layout {layout_query}/{layout_key}")
        dev = H.require_device(query, key, weights, block_table)
        self.lib = _lib.load()
        self.io = H.dtype_code(query.dtype, "query")
        if key.dtype != query.dtype:
            raise ValueError("query and key must share a dtype")
        self.wdt = H.dtype_code(weights.dtype, "weights", allow_f32=True)
        if layout_query == "TND":
            act_q = H.per_batch_from_cumsum(H.host_lengths(actual_seq_lengths_query))
            act_k = H.per_batch_from_cumsum(H.host_lengths(actual_seq_lengths_key))
            B = len(act_q)
            T1, N1, D = query.shape
            row_start = H.prefix(act_q)
            if row_start[-1] > T1:
                raise ValueError("actual_seq_lengths_query exceeds the packed query length")
            if is_pa:
                act_k = None   # per batch, not cumulative: set below
            elif layout_key == "TND":
                if sum(act_k) > key.shape[0]:
                    raise ValueError("actual_seq_lengths_key exceeds the packed key length")
                N2 = key.shape[1]
                key_start = H.prefix(act_k)[:-1]
                S2 = max(act_k) if act_k else 0
            else:
                N2, S2 = key.shape[2], key.shape[1]
                key_start = [b * S2 for b in range(B)]
            total_rows = T1
            out_lead = (T1,)
        else:
            B, S1, N1, D = query.shape
            act_q = H.host_lengths(actual_seq_lengths_query, B, S1)
            if not is_pa:
                _, S2, N2, _ = key.shape
                act_k = H.host_lengths(actual_seq_lengths_key, B, S2)
                key_start = [b * S2 for b in range(B)]
            row_start = [b * S1 for b in range(B + 1)]
            total_rows = B * S1
            out_lead = (B, S1)
        self.d_bt, self.max_blocks, self.page_bs, self.key_rows = None, 0, 0, 0
        if is_pa:
            # key cache [num_blocks, page, N2, D]; kv lengths per batch (as the SFA
            # forward's PA_BSND); S2 = max_blocks * page
            _, page, N2, _ = key.shape
            if block_table.dim() != 2 or block_table.shape[0] != B:
                raise ValueError("block_table must be [batch, max_blocks]")
            self.max_blocks, self.page_bs = int(block_table.shape[1]), int(page)
            S2 = self.max_blocks * self.page_bs
            act_k = H.host_lengths(actual_seq_lengths_key, B, S2)
            key_start = [0] * B
            self.key_rows = key.shape[0] * page
            self.d_bt = block_table.to(torch.int32).contiguous()
        if key.shape[-1] != D:
            raise ValueError("query and key head dims differ")
        if N1 % N2 != 0:
            raise ValueError(f"N1({N1}) must be divisible by N2({N2})")
        self.dev, self.B, self.N1, self.N2, self.D, self.S2 = dev, B, N1, N2, D, S2
        self.total_rows, self.k, self.sparse_mode = total_rows, int(sparse_count), sparse_mode
        self.act_q, self.act_k, self.row_start = act_q, act_k, row_start
        self.return_value = return_value
        self.q, self.kk, self.w = query.contiguous(), key.contiguous(), weights.contiguous()
        self.idx = torch.empty(out_lead + (N2, self.k), dtype=torch.int32, device=dev)
        self.vals = (torch.empty(out_lead + (N2, self.k), dtype=query.dtype, device=dev)
                     if return_value else torch.zeros(out_lead + (N2, self.k), dtype=query.dtype, device=dev))
        self.ld = _score_ld(S2)
        self.scores = torch.empty((max(total_rows, 1) * N2, self.ld), dtype=torch.int16, device=dev)
        tw = int(self.lib.dsa_li_topk_workspace_bytes(total_rows, N2, S2, self.k))
        self.topk_ws = torch.empty(tw, dtype=torch.uint8, device=dev) if tw > 0 else None
        self.d_row_start = H.i32(row_start, dev)
        self.d_key_start = H.i32(key_start, dev)
        self.d_aq = H.i32(act_q, dev)
        self.d_ak = H.i32(act_k, dev)
        self.max_rows = max(row_start[b + 1] - row_start[b] for b in range(B)) if B else 0
        self.max_kv = max(act_k) if act_k else 0

    def score(self):
        if self.total_rows == 0:
            return
        if self.d_bt is not None:
            _lib.check(self.lib.dsa_li_score_paged(
                self.q.data_ptr(), self.kk.data_ptr(), self.w.data_ptr(), self.io, self.wdt,
                self.d_row_start.data_ptr(), self.d_bt.data_ptr(), self.max_blocks, self.page_bs,
                self.key_rows, self.d_aq.data_ptr(), self.d_ak.data_ptr(), self.B, self.total_rows,
                self.N1, self.N2, self.D, self.max_rows, self.max_kv, self.sparse_mode,
                self.scores.data_ptr(), self.ld, H.stream_ptr(self.dev)), "dsa_li_score_paged")
            return
        _lib.check(self.lib.dsa_li_score(
            self.q.data_ptr(), self.kk.data_ptr(), self.w.data_ptr(), self.io, self.wdt,
            self.d_row_start.data_ptr(), self.d_key_start.data_ptr(), self.d_aq.data_ptr(),
            self.d_ak.data_ptr(), self.B, self.total_rows, self.N1, self.N2, self.D, self.S2,
            self.max_rows, self.max_kv, self.sparse_mode, self.scores.data_ptr(), self.ld,
            H.stream_ptr(self.dev)), "dsa_li_score")

    def topk(self):
        if self.total_rows == 0:
            return
        if self.topk_ws is not None:   # sparse_count above the LDS sort's cap
            _lib.check(self.lib.dsa_li_topk_ws(
                self.scores.data_ptr(), self.ld, self.io, self.d_row_start.data_ptr(),
                self.d_aq.data_ptr(), self.d_ak.data_ptr(), self.B, self.total_rows, self.N2, self.S2,
                self.sparse_mode, self.k, self.idx.data_ptr(),
                self.vals.data_ptr() if self.return_value else None, self.topk_ws.data_ptr(),
                self.topk_ws.numel(), H.stream_ptr(self.dev)), "dsa_li_topk_ws")
            return
        _lib.check(self.lib.dsa_li_topk(
            self.scores.data_ptr(), self.ld, self.io, self.d_row_start.data_ptr(),
            self.d_aq.data_ptr(), self.d_ak.data_ptr(), self.B, self.total_rows, self.N2, self.S2,
            self.sparse_mode, self.k, self.idx.data_ptr(),
            self.vals.data_ptr() if self.return_value else None, H.stream_ptr(self.dev)), "dsa_li_topk")

    def run(self):
        self.score()
        self.topk()
        return self.idx, self.vals


def lightning_indexer(query, key, weights, actual_seq_lengths_query=None,
                      actual_seq_lengths_key=None, block_table=None, layout_query="BSND",
                      layout_key="BSND", sparse_count=2048, sparse_mode=3, pre_tokens=INT64_MAX,
                      next_tokens=INT64_MAX, return_value=False):
    """MI355X lightning_indexer (indexer score + stable top-k).

    Args mirror lightning_indexer_triton.py:466-497: query [B,S1,N1,D] (BSND) or
    [T1,N1,D] (TND) fp16/bf16; key [B,S2,N2,D] / [T2,N2,D]; weights [B,S1,N1] /
    [T1,N1] fp16/bf16/fp32; actual_seq_lengths_* per-batch (BSND) or cumulative
    (TND); pre_tokens / next_tokens are ignored (as in the reference). Returns
    (indices, values). Beyond the reference (which raises on any block_table,
    :501-502): ``layout_key="PA_BSND"`` with ``block_table`` [B, max_blocks] reads the
    keys from a paged cache [num_blocks, block_size, N2, D] with per-batch kv lengths;
    any other layout with a block_table raises as the reference does."""
    return IndexerPlan(query, key, weights, actual_seq_lengths_query, actual_seq_lengths_key,
                       block_table, layout_query, layout_key, sparse_count, sparse_mode,
                       return_value).run()


class LightningIndexer(torch.nn.Module):
    """Module twin of ``LightningIndexerTriton`` (lightning_indexer_triton.py:420-463)."""

    def __init__(self, sparse_count=2048, sparse_mode=3, layout_query="BSND", layout_key="BSND",
                 return_value=False, pre_tokens=INT64_MAX, next_tokens=INT64_MAX):
        super().__init__()
        self.sparse_count = sparse_count
        self.sparse_mode = sparse_mode
        self.layout_query = layout_query
        self.layout_key = layout_key
        self.return_value = return_value
        self.pre_tokens = pre_tokens
        self.next_tokens = next_tokens

    def forward(self, query, key, weights, actual_seq_lengths_query=None,
                actual_seq_lengths_key=None, block_table=None):
        return lightning_indexer(query, key, weights,
                                 actual_seq_lengths_query=actual_seq_lengths_query,
                                 actual_seq_lengths_key=actual_seq_lengths_key,
                                 block_table=block_table, layout_query=self.layout_query,
                                 layout_key=self.layout_key, sparse_count=self.sparse_count,
                                 sparse_mode=self.sparse_mode, pre_tokens=self.pre_tokens,
                                 next_tokens=self.next_tokens, return_value=self.return_value)
