# SPDX-License-Identifier: Apache-2.0
"""Sparse indexer decode scoring on MI355X: FP8 paged MQA logits and the
top-k pool selection, the steps that produce the pool ids the kpool
expansion and the pooled attention consume.

The reference's decode indexer (integration/patch_decode_indexer.py:34-44)
calls vLLM's fp8_paged_mqa_logits_triton over the pool-granular context and
takes the top 512 pools per row (pool_topk, :64-72; expanded at
patch_indexer_sharding.py:58-79).  Neither function is in the reference; the
logits follow the published semantics of DeepGEMM's fp8_paged_mqa_logits:

    logits[t, j] = sum_h weights[t, h] * relu(s_j * (q[t, h] . k_j))

with q and the cached keys in FP8 E4M3 (OCP) and one fp32 scale per cached
key, the cache in DeepGEMM's fused layout (per page: block_size keys x 128
bytes, then block_size fp32 scales).  The selection keeps the k largest
logits of each row's valid positions, ties by position, and returns the
positions in ascending order.
"""
from __future__ import annotations

import torch

import _glm53_lib as _lib

HEAD_DIM = 128


def _fp8_bytes(q: torch.Tensor) -> torch.Tensor:
    if q.dtype == torch.uint8:
        return q
    if q.dtype == torch.float8_e4m3fn:
        return q.view(torch.uint8)
    raise ValueError(f"q must be float8_e4m3fn (or its uint8 bytes), got {q.dtype}")


def fp8_paged_mqa_logits(q: torch.Tensor, kv_cache: torch.Tensor, weights: torch.Tensor,
                         context_lens: torch.Tensor, block_tables: torch.Tensor, max_model_len: int,
                         clean_logits: bool = True) -> torch.Tensor:
    """q fp8 [B, next_n, H, 128]; kv_cache uint8 [num_blocks, block_size, 1, 132]
    (fused layout, page stride any multiple of 16 bytes); weights fp32
    [B * next_n, H]; context_lens int32 [B]; block_tables int32 [B, max_blocks].
    Returns fp32 logits [B * next_n, max_model_len].  Query i of request b sees
    positions j < context_lens[b] - next_n + 1 + i (next_n = 1 for decode)."""
    qb = _fp8_bytes(q)
    if qb.dim() != 4 or qb.shape[-1] != HEAD_DIM or qb.stride(-1) != 1:
        raise ValueError(f"q must be [B, next_n, H, {HEAD_DIM}] with contiguous rows, got {tuple(q.shape)}")
    B, next_n, H, _ = qb.shape
    if kv_cache.dim() != 4 or kv_cache.shape[-1] != HEAD_DIM + 4 or kv_cache.shape[2] != 1:
        raise ValueError(f"kv_cache must be [num_blocks, block_size, 1, {HEAD_DIM + 4}], got {tuple(kv_cache.shape)}")
    kvb = kv_cache if kv_cache.dtype == torch.uint8 else kv_cache.view(torch.uint8)
    nb, bs = kvb.shape[0], kvb.shape[1]
    if kvb.stride(1) != HEAD_DIM + 4 or kvb.stride(3) != 1:
        raise ValueError("kv_cache pages must be contiguous (stride between pages may be padded)")
    if weights.dtype != torch.float32 or tuple(weights.shape) != (B * next_n, H) or weights.stride(1) != 1:
        raise ValueError(f"weights must be fp32 [{B * next_n}, {H}]")
    if context_lens.dtype != torch.int32 or context_lens.numel() != B:
        raise ValueError("context_lens must be int32 [B]")
    if block_tables.dtype != torch.int32 or block_tables.dim() != 2 or block_tables.shape[0] != B:
        raise ValueError("block_tables must be int32 [B, max_blocks]")
    T = B * next_n
    qrows = qb.reshape(T, H, HEAD_DIM) if qb.is_contiguous() else qb.contiguous().reshape(T, H, HEAD_DIM)
    bt = block_tables if block_tables.stride(1) == 1 else block_tables.contiguous()
    ctx = context_lens.contiguous()
    if next_n > 1:   # one row per query token: its own causal length, its request's block table
        offs = torch.arange(next_n, device=ctx.device, dtype=torch.int32) - (next_n - 1)
        ctx = (ctx[:, None] + offs[None, :]).reshape(T).contiguous()
        bt = bt.repeat_interleave(next_n, dim=0).contiguous()
    logits = torch.empty((T, max_model_len), dtype=torch.float32, device=q.device)
    if T == 0 or max_model_len == 0:
        return logits
    L = _lib.load()
    with torch.cuda.device(q.device):
        rc = L.glm53_fp8_paged_mqa_logits(qrows.data_ptr(), qrows.stride(0), qrows.stride(1), kvb.data_ptr(),
                                          kvb.stride(0), bs, nb, weights.data_ptr(), weights.stride(0),
                                          ctx.data_ptr(), bt.data_ptr(), bt.stride(0), bt.shape[1], T, H,
                                          HEAD_DIM, max_model_len, int(bool(clean_logits)), logits.data_ptr(),
                                          logits.stride(0), _lib.stream_handle(q.device))
    _lib.check(rc, "glm53_fp8_paged_mqa_logits")
    return logits


def indexer_topk(logits: torch.Tensor, lengths: torch.Tensor, k: int = 512) -> torch.Tensor:
    """The k largest logits of each row among positions [0, lengths[r]):
    int32 [rows, k] positions in ascending order (-1 padding when a row has
    fewer than k valid positions)."""
    if logits.dtype != torch.float32 or logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be fp32 [rows, n] with contiguous rows")
    rows, n = logits.shape
    if lengths.dtype != torch.int32 or lengths.numel() != rows:
        raise ValueError("lengths must be int32 [rows]")
    if not 1 <= k <= n:
        raise ValueError(f"1 <= k <= {n} required, got {k}")
    out = torch.empty((rows, k), dtype=torch.int32, device=logits.device)
    if rows == 0:
        return out
    L = _lib.load()
    ws_bytes = int(L.glm53_indexer_topk_workspace_bytes(rows, n, k))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=logits.device)
    with torch.cuda.device(logits.device):
        rc = L.glm53_indexer_topk(logits.data_ptr(), logits.stride(0), lengths.contiguous().data_ptr(), rows, n, k,
                                  ws.data_ptr(), ws_bytes, out.data_ptr(), out.stride(0),
                                  _lib.stream_handle(logits.device))
    _lib.check(rc, "glm53_indexer_topk")
    return out


def indexer_decode_pool_topk(q: torch.Tensor, kv_cache: torch.Tensor, weights: torch.Tensor,
                             context_lens: torch.Tensor, block_tables: torch.Tensor, max_model_len: int,
                             k: int = 512) -> torch.Tensor:
    """Decode indexer: logits over the pool-granular context, then the top-k
    pools of each query (int32 [B * next_n, k], ascending, -1 padded) -- the
    pool_topk the kpool expansion (sparse_utils.expand_pools_and_append_tail)
    or titan_mla.triton_mla_sparse_attention_pooled consumes."""
    logits = fp8_paged_mqa_logits(q, kv_cache, weights, context_lens, block_tables, max_model_len,
                                  clean_logits=False)
    B, next_n = q.shape[0], q.shape[1]
    lens = context_lens.to(torch.int32)
    cap = block_tables.shape[1] * kv_cache.shape[1]
    if next_n == 1 and min(max_model_len, cap) >= k:
        # the top-k clamps each row's length to the columns it is given: the
        # columns the block table can hold (no separate clamp launch)
        return indexer_topk(logits[:, :min(max_model_len, cap)], lens.contiguous(), k)
    if next_n > 1:
        offs = torch.arange(next_n, device=lens.device, dtype=torch.int32) - (next_n - 1)
        lens = (lens[:, None] + offs[None, :]).reshape(-1)
    # positions the block table cannot hold were not scored (clean_logits=False)
    lens = torch.clamp(lens, max=cap)
    return indexer_topk(logits, lens.to(torch.int32).contiguous(), k)
