# SPDX-License-Identifier: Apache-2.0
"""Sparse NoPE MLA attention over the per-token INT8 cache, MI355X HIP kernels.

Drop-in for `triton_mla_sparse_attention` of kernels/titan_mla.py:452-581
(same name, signature, assertions and return value).  The kernels live in
csrc/sparse_mla.hip behind glm53_sparse_mla; they run on the caller's
current stream without host synchronisation, so the call is
graph-capturable.  Output and split workspace come from torch's caching
allocator.

Cache rows are 528 bytes: 512 int8 latents, fp32 scale at byte 512, zero
padding; the latent serves as both K and V (NoPE, one KV head).  The RoPE
(dim_qk = 576) and BF16-cache branches the reference inherits are not part of
its tested contract and are not provided here.
"""
import functools

import torch

import _glm53_lib as _lib

LOG2E = 1.4426950408889634
LOGE2 = 0.6931471805599453

_BLOCK_DMODEL = 512
_BLOCK_DPE = 64
_BLOCK_DV = 512
_DIM_QK = _BLOCK_DMODEL + _BLOCK_DPE  # 576
_BLOCK_H = 16
_ROW_BYTES = 528
# Smallest tile width of the reference's autotune space: top-k must be a
# multiple of it (kernels/titan_mla.py:45-49, :485-488).
_MIN_BLOCK_N = 32
KV_SPLITS_CANDIDATES = (1, 2, 4, 8, 16)
_MIN_TOPK_PER_SPLIT = 128
_SPLIT_MAX_OCCUPANCY = 4
# Query tokens per library call (the split kernel's grid y); larger calls are
# cut into consecutive token ranges.
_MAX_TOKENS_PER_CALL = 65535


def num_compute_units(device_index):
    return torch.cuda.get_device_properties(device_index).multi_processor_count


def _next_power_of_2(n: int) -> int:
    return 1 << (n - 1).bit_length() if n > 0 else 1


@functools.lru_cache(maxsize=256)
def _choose_num_kv_splits(num_tokens: int, num_head_groups: int, index_topk: int,
                          sm_count: int) -> int:
    """Power-of-2 split count that fills the device without dropping per-split
    work below _MIN_TOPK_PER_SPLIT indices; 1 when the single-pass grid already
    covers a quarter of the compute units (kernels/titan_mla.py:432-449)."""
    baseline = num_tokens * num_head_groups
    if baseline == 0 or baseline * _SPLIT_MAX_OCCUPANCY >= sm_count:
        return 1
    ideal = _next_power_of_2(max(1, index_topk // _MIN_TOPK_PER_SPLIT))
    max_splits = max(1, sm_count // baseline)
    max_splits = 1 << (max_splits.bit_length() - 1)
    num_kv_splits = min(ideal, max_splits)
    while num_kv_splits > 1 and index_topk % num_kv_splits != 0:
        num_kv_splits //= 2
    return max(1, num_kv_splits)


@functools.lru_cache(maxsize=256)
def _choose_num_kv_splits_mi355x(num_tokens: int, num_head_groups: int, index_topk: int,
                                 cu_count: int) -> int:
    """Split count used when the caller leaves num_kv_splits to the library.

    The split kernel runs one workgroup per (split, token, head group), one
    key group of four waves per tile of a round, and one workgroup fits a
    compute unit (up to ~136 KB of LDS).  Decode latency is set by the
    per-workgroup chain (index load -> row gather -> tiles), so the split
    count is capped where every workgroup still starts in the first wave
    (tokens * groups * splits <= CUs) and, with more than one (token, head
    group) unit, each split has two 32-key tiles (the merge reads every
    split's partials, so more units call for fewer, longer splits); under
    the cap it takes the fewest tiles per split, then the fewest splits that
    give that many.  At 2176 indices: B=1 68 one-tile splits (9.35 us warm
    against 10.1-10.5 us for 34 of two), B=2 and B=4 34 splits of 2 tiles
    (B=2 at 68: 10.9 against 10.4 us), B=8 23 splits of 3 (13.1 us per step
    over a 5-layer rotation against 13.4 us for 17 of 4).  (The reference's
    _choose_num_kv_splits targets Triton on 70 SMs and is kept above,
    unchanged, for callers that want its exact answers.)  Batches of 5-7
    tokens with one head group are sized as 8: the library numbers them as
    8 tokens so that each token's splits share one XCD (23 splits: B=7 11.31
    us against 12.03 us for 34 splits spread over every XCD).
    """
    base = num_tokens * num_head_groups
    if num_head_groups == 1 and 5 <= num_tokens <= 7:
        base = 8
    if base == 0 or index_topk <= 0 or index_topk % _MIN_BLOCK_N:
        return 1
    tiles = index_topk // _MIN_BLOCK_N
    min_tiles = 1 if base == 1 else 2
    cap = max(1, min(cu_count // base, tiles // min_tiles))
    per_split = -(-tiles // cap)
    return -(-tiles // per_split)


def triton_mla_sparse_attention(
    q: torch.Tensor,
    kv: torch.Tensor,
    indices: torch.Tensor,
    sm_scale: float,
    num_kv_splits: int | None = None,
    sm_count: int | None = None,
) -> torch.Tensor:
    """Sparse MLA attention over top-k indices.

    Args:
        q:         [num_tokens, num_heads_q, 512] bf16
        kv:        [seq_kv, 1, 528] int8 packed cache rows
        indices:   [num_tokens, 1, topk] int32; entries outside [0, seq_kv)
                   are masked
        sm_scale:  softmax scale
        num_kv_splits: None/0 = heuristic, 1 = single pass, n = n splits
        sm_count:  compute-unit count for the heuristic (queried if None);
                   the split policy is _choose_num_kv_splits_mi355x

    Returns:
        out: [num_tokens, num_heads_q, 512] bf16
    """
    num_tokens, num_heads_q, dim_qk = q.shape
    assert dim_qk in (_BLOCK_DMODEL, _DIM_QK), (
        f"sparse MLA kernel requires dim_qk={_BLOCK_DMODEL} (NoPE) or "
        f"{_DIM_QK} (RoPE), got {dim_qk}"
    )
    assert kv.shape[1] == 1 and kv.shape[2] == (_ROW_BYTES if kv.dtype == torch.int8 else dim_qk)
    index_topk = indices.shape[2]
    assert index_topk % _MIN_BLOCK_N == 0, (
        f"topk ({index_topk}) must be a multiple of the smallest autotune "
        f"BLOCK_N ({_MIN_BLOCK_N})"
    )
    if dim_qk != _BLOCK_DMODEL or kv.dtype != torch.int8:
        raise NotImplementedError("only the NoPE INT8-cache path (dim_qk=512, 528-byte rows) is built")
    if q.dtype != torch.bfloat16:
        raise ValueError(f"q must be bf16, got {q.dtype}")

    num_head_groups = triton_cdiv(num_heads_q, min(_BLOCK_H, num_heads_q))
    if num_kv_splits is None or num_kv_splits == 0:
        if sm_count is None:
            sm_count = num_compute_units(q.device.index)
        num_kv_splits = _choose_num_kv_splits_mi355x(num_tokens, num_head_groups, index_topk, sm_count)
    if num_kv_splits < 1:
        raise ValueError(f"num_kv_splits must be >= 1, got {num_kv_splits}")

    out = torch.empty((num_tokens, num_heads_q, _BLOCK_DV), dtype=torch.bfloat16, device=q.device)
    if num_tokens == 0:
        return out
    if num_tokens > _MAX_TOKENS_PER_CALL:
        for t0 in range(0, num_tokens, _MAX_TOKENS_PER_CALL):
            t1 = min(t0 + _MAX_TOKENS_PER_CALL, num_tokens)
            out[t0:t1] = triton_mla_sparse_attention(q[t0:t1], kv, indices[t0:t1], sm_scale, num_kv_splits)
        return out

    if q.stride(2) != 1 or q.stride(1) % 8 or q.stride(0) % 8 or q.data_ptr() % 16:
        q = q.contiguous()
    if indices.dtype != torch.int32:
        # Out-of-range wide indices stay masked after narrowing.
        valid = (indices >= 0) & (indices < kv.shape[0])
        indices = torch.where(valid, indices, torch.full_like(indices, -1)).to(torch.int32)
    if indices.stride(2) != 1:
        indices = indices.contiguous()

    L = _lib.load()
    ws_bytes = L.glm53_sparse_mla_workspace_bytes(num_tokens, num_heads_q, num_kv_splits)
    workspace = (torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes > 0 else None)
    with torch.cuda.device(q.device):
        rc = L.glm53_sparse_mla(
            q.data_ptr(), q.stride(0), q.stride(1),
            kv.data_ptr(), kv.stride(0), kv.shape[0],
            indices.data_ptr(), indices.stride(0),
            num_tokens, num_heads_q, index_topk,
            float(sm_scale), num_kv_splits,
            workspace.data_ptr() if workspace is not None else None, ws_bytes,
            out.data_ptr(), out.stride(0), out.stride(1),
            _lib.stream_handle(q.device))
    _lib.check(rc, "glm53_sparse_mla")
    return out


def triton_mla_sparse_attention_paged(
    q: torch.Tensor,
    kv_cache: torch.Tensor,
    req_indices: torch.Tensor,
    req_id_per_token: torch.Tensor,
    block_table: torch.Tensor,
    sm_scale: float,
    num_kv_splits: int | None = None,
    sm_count: int | None = None,
) -> torch.Tensor:
    """The adapter's two steps in one launch (integration/titan_backend.py:48-54):
    request-relative indices are mapped to cache rows as
    sparse_utils.triton_convert_req_index_to_global_index maps them, inside
    the attention's index load.  Same result as converting first and calling
    triton_mla_sparse_attention on sparse_utils.flat_kv_row_view(kv_cache)
    whenever that view exists; the page stride here may be any multiple of
    16 bytes (pages padded to an alignment), which the flat view cannot
    express.

    Args:
        q:            [T, H, 512] bf16
        kv_cache:     int8 [num_blocks, block_size, 528] paged cache (row and
                      page strides multiples of 16 bytes)
        req_indices:  int32 [T, topk] or [T, 1, topk] request-relative token
                      positions, -1 for padding
        req_id_per_token: int32 [T]
        block_table:  int32 [num_reqs, max_blocks]
    """
    assert kv_cache.dtype == torch.int8 and kv_cache.dim() == 3 and kv_cache.shape[2] == _ROW_BYTES
    assert kv_cache.stride(2) == 1
    if req_indices.dim() == 3:
        assert req_indices.shape[1] == 1
        req_indices = req_indices[:, 0, :]
    assert req_indices.dtype == torch.int32 and req_id_per_token.dtype == torch.int32
    assert block_table.dtype == torch.int32 and block_table.dim() == 2
    num_tokens, num_heads_q, dim_qk = q.shape
    assert dim_qk == _BLOCK_DMODEL and q.dtype == torch.bfloat16
    assert req_id_per_token.numel() == num_tokens and req_indices.shape[0] == num_tokens
    index_topk = req_indices.shape[1]
    assert index_topk % _MIN_BLOCK_N == 0, (
        f"topk ({index_topk}) must be a multiple of the smallest autotune BLOCK_N ({_MIN_BLOCK_N})")

    num_head_groups = triton_cdiv(num_heads_q, min(_BLOCK_H, num_heads_q))
    if num_kv_splits is None or num_kv_splits == 0:
        if sm_count is None:
            sm_count = num_compute_units(q.device.index)
        num_kv_splits = _choose_num_kv_splits_mi355x(num_tokens, num_head_groups, index_topk, sm_count)
    if num_kv_splits < 1:
        raise ValueError(f"num_kv_splits must be >= 1, got {num_kv_splits}")
    out = torch.empty((num_tokens, num_heads_q, _BLOCK_DV), dtype=torch.bfloat16, device=q.device)
    if num_tokens == 0:
        return out
    if num_tokens > _MAX_TOKENS_PER_CALL:
        for t0 in range(0, num_tokens, _MAX_TOKENS_PER_CALL):
            t1 = min(t0 + _MAX_TOKENS_PER_CALL, num_tokens)
            out[t0:t1] = triton_mla_sparse_attention_paged(q[t0:t1], kv_cache, req_indices[t0:t1],
                                                           req_id_per_token[t0:t1], block_table, sm_scale,
                                                           num_kv_splits)
        return out
    if q.stride(2) != 1 or q.stride(1) % 8 or q.stride(0) % 8 or q.data_ptr() % 16:
        q = q.contiguous()
    if req_indices.stride(1) != 1:
        req_indices = req_indices.contiguous()
    if block_table.stride(1) != 1:
        block_table = block_table.contiguous()
    req_id_per_token = req_id_per_token.contiguous()

    L = _lib.load()
    ws_bytes = L.glm53_sparse_mla_workspace_bytes(num_tokens, num_heads_q, num_kv_splits)
    workspace = (torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes > 0 else None)
    with torch.cuda.device(q.device):
        rc = L.glm53_sparse_mla_paged(
            q.data_ptr(), q.stride(0), q.stride(1),
            kv_cache.data_ptr(), kv_cache.stride(0), kv_cache.stride(1), kv_cache.shape[0],
            req_indices.data_ptr(), req_indices.stride(0),
            req_id_per_token.data_ptr(),
            block_table.data_ptr() if block_table.numel() else None,
            block_table.shape[0], block_table.stride(0), block_table.shape[1],
            kv_cache.shape[1],
            num_tokens, num_heads_q, index_topk,
            float(sm_scale), num_kv_splits,
            workspace.data_ptr() if workspace is not None else None, ws_bytes,
            out.data_ptr(), out.stride(0), out.stride(1),
            _lib.stream_handle(q.device))
    _lib.check(rc, "glm53_sparse_mla_paged")
    return out


def triton_mla_sparse_attention_pooled(
    q: torch.Tensor,
    kv_cache: torch.Tensor,
    pool_ids: torch.Tensor,
    seq_lens: torch.Tensor | None,
    pool_size: int,
    req_id_per_token: torch.Tensor,
    block_table: torch.Tensor,
    sm_scale: float,
    topk: int = 2176,
    num_kv_splits: int | None = None,
    sm_count: int | None = None,
) -> torch.Tensor:
    """Indexer output straight to attention: slot k of token t's topk index
    slots is the position sparse_utils.expand_pools_and_append_tail (or
    expand_pools_to_tokens when seq_lens is None) puts there, -1 past the
    expansion, and the positions are resolved through the block table as in
    triton_mla_sparse_attention_paged.  One launch replaces expansion,
    conversion and the attention's split kernel; the output equals
    expanding into a -1-filled [T, topk] buffer and calling the paged
    attention.

    Args:
        pool_ids:  int32 [T, num_pools] request-relative pool ids (-1 invalid)
        seq_lens:  int32 [T] query sequence lengths (position + 1), or None
        topk:      index slots (multiple of 32, >= the expanded width)
    """
    assert kv_cache.dtype == torch.int8 and kv_cache.dim() == 3 and kv_cache.shape[2] == _ROW_BYTES
    assert kv_cache.stride(2) == 1
    assert pool_ids.dtype == torch.int32 and pool_ids.dim() == 2
    assert req_id_per_token.dtype == torch.int32 and block_table.dtype == torch.int32 and block_table.dim() == 2
    num_tokens, num_heads_q, dim_qk = q.shape
    assert dim_qk == _BLOCK_DMODEL and q.dtype == torch.bfloat16
    assert pool_ids.shape[0] == num_tokens and req_id_per_token.numel() == num_tokens
    assert topk % _MIN_BLOCK_N == 0, f"topk ({topk}) must be a multiple of {_MIN_BLOCK_N}"
    assert pool_size >= 1
    width = pool_ids.shape[1] * pool_size + (pool_size - 1 if seq_lens is not None else 0)
    assert topk >= width, f"topk ({topk}) is narrower than the expansion ({width})"

    num_head_groups = triton_cdiv(num_heads_q, min(_BLOCK_H, num_heads_q))
    if num_kv_splits is None or num_kv_splits == 0:
        if sm_count is None:
            sm_count = num_compute_units(q.device.index)
        num_kv_splits = _choose_num_kv_splits_mi355x(num_tokens, num_head_groups, topk, sm_count)
    if num_kv_splits < 1:
        raise ValueError(f"num_kv_splits must be >= 1, got {num_kv_splits}")
    out = torch.empty((num_tokens, num_heads_q, _BLOCK_DV), dtype=torch.bfloat16, device=q.device)
    if num_tokens == 0:
        return out
    if num_tokens > _MAX_TOKENS_PER_CALL:
        for t0 in range(0, num_tokens, _MAX_TOKENS_PER_CALL):
            t1 = min(t0 + _MAX_TOKENS_PER_CALL, num_tokens)
            out[t0:t1] = triton_mla_sparse_attention_pooled(
                q[t0:t1], kv_cache, pool_ids[t0:t1], seq_lens[t0:t1] if seq_lens is not None else None,
                pool_size, req_id_per_token[t0:t1], block_table, sm_scale, topk, num_kv_splits)
        return out
    if q.stride(2) != 1 or q.stride(1) % 8 or q.stride(0) % 8 or q.data_ptr() % 16:
        q = q.contiguous()
    if pool_ids.stride(1) != 1:
        pool_ids = pool_ids.contiguous()
    if seq_lens is not None:
        assert seq_lens.numel() == num_tokens
        seq_lens = seq_lens.to(torch.int32).contiguous()
    if block_table.stride(1) != 1:
        block_table = block_table.contiguous()
    req_id_per_token = req_id_per_token.contiguous()

    L = _lib.load()
    ws_bytes = L.glm53_sparse_mla_workspace_bytes(num_tokens, num_heads_q, num_kv_splits)
    workspace = (torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes > 0 else None)
    with torch.cuda.device(q.device):
        rc = L.glm53_sparse_mla_pooled(
            q.data_ptr(), q.stride(0), q.stride(1),
            kv_cache.data_ptr(), kv_cache.stride(0), kv_cache.stride(1), kv_cache.shape[0],
            pool_ids.data_ptr(), pool_ids.stride(0), pool_ids.shape[1],
            seq_lens.data_ptr() if seq_lens is not None else None, pool_size,
            req_id_per_token.data_ptr(),
            block_table.data_ptr() if block_table.numel() else None,
            block_table.shape[0], block_table.stride(0), block_table.shape[1],
            kv_cache.shape[1],
            num_tokens, num_heads_q, topk,
            float(sm_scale), num_kv_splits,
            workspace.data_ptr() if workspace is not None else None, ws_bytes,
            out.data_ptr(), out.stride(0), out.stride(1),
            _lib.stream_handle(q.device))
    _lib.check(rc, "glm53_sparse_mla_pooled")
    return out


def sparse_mla_partials(q, kv, indices, sm_scale, num_kv_splits):
    """First stage only: per-split normalised outputs and LSEs (fp32) in one
    buffer laid out as glm53.h documents (part [T*S*Hp, 512] then lse
    [T*S*Hp], Hp = heads rounded up to 16).  For callers that merge splits
    themselves, e.g. after gathering one token's splits from several devices."""
    assert q.dim() == 3 and q.shape[2] == _BLOCK_DMODEL and q.dtype == torch.bfloat16
    assert kv.dtype == torch.int8 and kv.shape[1] == 1 and kv.shape[2] == _ROW_BYTES
    assert indices.dtype == torch.int32 and indices.stride(2) == 1
    if q.stride(2) != 1 or q.stride(1) % 8 or q.stride(0) % 8 or q.data_ptr() % 16:
        q = q.contiguous()
    T, H, _ = q.shape
    L = _lib.load()
    nbytes = L.glm53_sparse_mla_partials_bytes(T, H, num_kv_splits)
    buf = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=q.device)
    with torch.cuda.device(q.device):
        rc = L.glm53_sparse_mla_partials(q.data_ptr(), q.stride(0), q.stride(1), kv.data_ptr(), kv.stride(0),
                                         kv.shape[0], indices.data_ptr(), indices.stride(0), T, H,
                                         indices.shape[2], float(sm_scale), num_kv_splits, buf.data_ptr(),
                                         nbytes, _lib.stream_handle(q.device))
    _lib.check(rc, "glm53_sparse_mla_partials")
    return buf


def sparse_mla_gather_floor(q, kv, indices, num_kv_splits, out=None):
    """Diagnostic: the memory chain of sparse_mla_partials alone (the same
    grid, index loads, row gathers and partial stores, no arithmetic; the
    buffer then holds junk) -- the floor under the split kernel's time.
    Decode splits only (at most 256 indices per split)."""
    assert q.dim() == 3 and q.shape[2] == _BLOCK_DMODEL and q.dtype == torch.bfloat16 and q.is_contiguous()
    assert kv.dtype == torch.int8 and kv.shape[1] == 1 and kv.shape[2] == _ROW_BYTES
    assert indices.dtype == torch.int32 and indices.stride(2) == 1
    T, H, _ = q.shape
    L = _lib.load()
    nbytes = L.glm53_sparse_mla_partials_bytes(T, H, num_kv_splits)
    buf = out if out is not None else torch.empty(max(nbytes, 16), dtype=torch.uint8, device=q.device)
    with torch.cuda.device(q.device):
        rc = L.glm53_sparse_mla_gather_floor(q.data_ptr(), q.stride(0), q.stride(1), kv.data_ptr(), kv.stride(0),
                                             kv.shape[0], indices.data_ptr(), indices.stride(0), T, H,
                                             indices.shape[2], num_kv_splits, buf.data_ptr(), nbytes,
                                             _lib.stream_handle(q.device))
    _lib.check(rc, "glm53_sparse_mla_gather_floor")
    return buf


def sparse_mla_merge(partials, num_tokens, num_heads, num_kv_splits):
    """Second stage: log-sum-exp merge of sparse_mla_partials' buffer."""
    out = torch.empty((num_tokens, num_heads, _BLOCK_DV), dtype=torch.bfloat16, device=partials.device)
    L = _lib.load()
    with torch.cuda.device(partials.device):
        rc = L.glm53_sparse_mla_merge(partials.data_ptr(), partials.numel(), num_tokens, num_heads,
                                      num_kv_splits, out.data_ptr(), out.stride(0), out.stride(1),
                                      _lib.stream_handle(partials.device))
    _lib.check(rc, "glm53_sparse_mla_merge")
    return out


def triton_cdiv(a: int, b: int) -> int:
    return (a + b - 1) // b
