# SPDX-License-Identifier: Apache-2.0
"""MI355X versions of the two vLLM sparse-MLA helpers the reference's adapter
calls before the attention (integration/titan_backend.py:48-52):

    rows, stride = flat_kv_row_view(kv_cache, block_size)
    indices = triton_convert_req_index_to_global_index(
        req_id_per_token, block_table, indices,
        BLOCK_SIZE=block_size, BLOCK_STRIDE_ROWS=stride, NUM_TOPK_TOKENS=topk)

They come from vLLM's v1/attention/backends/mla/sparse_utils.py at the
revision the reference pins, which is not available here; the mapping below is
the one glm53.h documents (a position p of a token of request r maps to
block_table[r, p // BLOCK_SIZE] * BLOCK_STRIDE_ROWS + p % BLOCK_SIZE, and to
-1 when p < 0 or its block lies beyond the table).  Both run on the GPU;
titan_mla.triton_mla_sparse_attention_paged fuses the conversion into the
attention gather.

Also here: the indexer's kpool expansion (expand_pools_and_append_tail,
expand_pools_to_tokens: top-k pool ids -> token positions), the step before
the conversion; titan_mla.triton_mla_sparse_attention_pooled fuses both into
the attention gather.
"""
import torch

import _glm53_lib as _lib


def flat_kv_row_view(kv_cache: torch.Tensor, block_size: int):
    """Flat row view of a paged cache.

    kv_cache: [num_blocks, block_size, row_width] with contiguous rows; the
    page (block) stride may be padded but must be a whole number of rows.
    Returns (rows, stride): rows is a [(num_blocks - 1) * stride + block_size,
    row_width] view whose row b * stride + i is row i of block b, and stride is
    the row count of one padded page (BLOCK_STRIDE_ROWS).
    """
    if kv_cache.dim() != 3:
        raise ValueError(f"expected a [num_blocks, block_size, width] cache, got {tuple(kv_cache.shape)}")
    nb, bs, width = kv_cache.shape
    if bs != block_size:
        raise ValueError(f"cache block size {bs} != block_size {block_size}")
    if kv_cache.stride(2) != 1 or kv_cache.stride(1) != width or kv_cache.stride(0) % width:
        raise ValueError("rows must be contiguous and the page stride a whole number of rows")
    stride = kv_cache.stride(0) // width
    n_rows = (nb - 1) * stride + bs if nb > 0 else 0
    rows = torch.as_strided(kv_cache, (n_rows, width), (width, 1))
    return rows, stride


def triton_convert_req_index_to_global_index(
    req_id: torch.Tensor,
    block_table: torch.Tensor,
    token_indices: torch.Tensor,
    BLOCK_SIZE: int = 64,
    NUM_TOPK_TOKENS: int = 2048,
    BLOCK_N: int = 128,
    BLOCK_STRIDE_ROWS: int | None = None,
    HAS_PREFILL_WORKSPACE: bool = False,
    **kwargs,
) -> torch.Tensor:
    """Request-relative token positions -> flat cache rows (int32, same shape
    as token_indices).  req_id: int32 [T]; block_table: int32 [R, max_blocks];
    token_indices: int32 [T, NUM_TOPK_TOKENS], -1 for padding.  BLOCK_N is
    accepted for signature compatibility (the HIP kernel covers 256 indices per
    workgroup).  The prefill-workspace options of later vLLM revisions are not
    provided."""
    if HAS_PREFILL_WORKSPACE or any(v is not None and v is not False for v in kwargs.values()):
        raise NotImplementedError("prefill-workspace index conversion is not provided")
    assert req_id.dtype == torch.int32 and block_table.dtype == torch.int32
    assert token_indices.dtype == torch.int32
    assert token_indices.dim() == 2 and token_indices.shape[1] == NUM_TOPK_TOKENS
    assert req_id.numel() == token_indices.shape[0]
    stride_rows = BLOCK_SIZE if BLOCK_STRIDE_ROWS is None else BLOCK_STRIDE_ROWS
    if token_indices.stride(1) != 1:
        token_indices = token_indices.contiguous()
    if block_table.dim() != 2 or block_table.stride(1) != 1:
        block_table = block_table.reshape(block_table.shape[0], -1).contiguous()
    req_id = req_id.contiguous()
    out = torch.empty_like(token_indices, memory_format=torch.contiguous_format)
    T, topk = token_indices.shape
    if T == 0 or topk == 0:
        return out
    L = _lib.load()
    with torch.cuda.device(token_indices.device):
        rc = L.glm53_convert_req_index(
            req_id.data_ptr(), block_table.data_ptr() if block_table.numel() else None,
            block_table.shape[0], block_table.stride(0), block_table.shape[1],
            token_indices.data_ptr(), token_indices.stride(0), out.data_ptr(), out.stride(0),
            T, topk, BLOCK_SIZE, stride_rows, _lib.stream_handle(token_indices.device))
    _lib.check(rc, "glm53_convert_req_index")
    return out


def _expand(pool_ids: torch.Tensor, seq_lens, pool_size: int, out_cols: int) -> torch.Tensor:
    assert pool_ids.dim() == 2 and pool_ids.dtype in (torch.int32, torch.int64)
    if pool_ids.stride(1) != 1:
        pool_ids = pool_ids.contiguous()
    rows, num_pools = pool_ids.shape
    out = torch.empty((rows, out_cols), dtype=torch.int32, device=pool_ids.device)
    if rows == 0 or out_cols == 0:
        return out
    if seq_lens is not None:
        seq_lens = seq_lens.to(torch.int32).contiguous()
        assert seq_lens.numel() == rows
    L = _lib.load()
    with torch.cuda.device(pool_ids.device):
        rc = L.glm53_expand_pools(pool_ids.data_ptr(), int(pool_ids.dtype == torch.int64), pool_ids.stride(0),
                                  num_pools, seq_lens.data_ptr() if seq_lens is not None else None, pool_size,
                                  out.data_ptr(), out.stride(0), rows, out_cols,
                                  _lib.stream_handle(pool_ids.device))
    _lib.check(rc, "glm53_expand_pools")
    return out


def expand_pools_and_append_tail(pool_ids: torch.Tensor, seq_lens: torch.Tensor, pool_size: int) -> torch.Tensor:
    """The indexer's kpool expansion with the tail pool (the operation the
    reference's sharding patch calls, integration/patch_indexer_sharding.py:
    92-94; CPU model tests/verify_indexer_sharding.py:72-79): row t becomes
    pool_ids[t, j] * pool_size + o for every pool j and offset o (-1 for a
    negative id), then the pool_size - 1 tail slots seq_lens[t] // pool_size
    * pool_size + j for j < seq_lens[t] % pool_size (-1 otherwise).
    Returns int32 [rows, num_pools * pool_size + pool_size - 1]."""
    return _expand(pool_ids, seq_lens, pool_size, pool_ids.shape[1] * pool_size + pool_size - 1)


def expand_pools_to_tokens(pool_ids: torch.Tensor, valid: torch.Tensor, topk_tokens: int,
                           pool_size: int) -> torch.Tensor:
    """The expansion without a tail (no positions; patch_indexer_sharding.py:
    97-99).  Pools where `valid` is False count as -1.  Returns int32
    [rows, topk_tokens] (topk_tokens = num_pools * pool_size)."""
    assert topk_tokens == pool_ids.shape[1] * pool_size
    if valid is not None:
        pool_ids = torch.where(valid, pool_ids, torch.full_like(pool_ids, -1))
    return _expand(pool_ids, None, pool_size, topk_tokens)
