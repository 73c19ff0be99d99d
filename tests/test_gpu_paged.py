"""GPU parity of the request-relative index path: the standalone conversion
(sparse_utils.triton_convert_req_index_to_global_index) bit-exact against the
oracle's conversion, and the fused paged attention
(titan_mla.triton_mla_sparse_attention_paged) bit-identical to converting
first and calling triton_mla_sparse_attention on the flat row view, and
within the attention bar of the oracle over each request's logically ordered
cache.  vLLM's own helper is not available here: parity with it is unpinned
beyond the mapping glm53.h documents."""
import numpy as np
import pytest
import torch

import workloads as W
from conftest import log_case

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def paged_cache(cuda, num_blocks, block_size, page_rows, seed):
    """int8 [num_blocks, block_size, 528] view of pages of page_rows rows,
    filled by store_int8 through its slot mapping; returns the view and the
    flat rows as numpy (padding rows included)."""
    from titan_kv import store_int8
    from sparse_utils import flat_kv_row_view
    g = W.gen(cuda, seed)
    raw = torch.zeros(num_blocks, page_rows, 528, dtype=torch.int8, device=cuda)
    cache = raw[:, :block_size, :]
    n = num_blocks * block_size
    x = torch.randn(n, 512, generator=g, device=cuda).to(torch.bfloat16)
    store_int8(x, cache, torch.arange(n, device=cuda))
    torch.cuda.synchronize()
    rows, stride = flat_kv_row_view(cache, block_size)
    assert stride == page_rows
    return cache, rows, rows.contiguous().view(torch.uint8).cpu().numpy()


def tables(cuda, num_reqs, max_blocks, num_blocks, seed):
    rng = np.random.default_rng(seed)
    bt = rng.permutation(num_blocks)[: num_reqs * max_blocks].reshape(num_reqs, max_blocks)
    return torch.as_tensor(bt.astype(np.int32), device=cuda)


@pytest.mark.parametrize("block_size,page_rows,max_blocks,num_blocks",
                         [(64, 64, 40, 128), (64, 66, 40, 128), (2304, 2304, 3, 10), (256, 257, 9, 40)])
def test_convert_matches_oracle(cuda, oracle, block_size, page_rows, max_blocks, num_blocks):
    from sparse_utils import triton_convert_req_index_to_global_index as conv
    log_case("convert", block_size, page_rows, max_blocks)
    g = W.gen(cuda, 21)
    bt = tables(cuda, 3, max_blocks, num_blocks, 5)
    T, topk = 9, 2176
    req = torch.tensor([0, 1, 2, 1, 0, 3, -1, 2, 0], dtype=torch.int32, device=cuda)   # 3, -1: no table row
    span = max_blocks * block_size
    idx = torch.randint(-5, span + 300, (T, topk), generator=g, device=cuda, dtype=torch.int32)
    idx[:, -100:] = -1
    out = conv(req, bt, idx, BLOCK_SIZE=block_size, NUM_TOPK_TOKENS=topk, BLOCK_STRIDE_ROWS=page_rows)
    torch.cuda.synchronize()
    want = oracle.convert_req_index(req.cpu().numpy(), bt.cpu().numpy(), idx.cpu().numpy(), block_size, page_rows)
    assert np.array_equal(out.cpu().numpy(), want)
    # wrapping products (garbage table entries) follow int32 arithmetic
    big = torch.full((1, 4), 2 ** 30 + 7, dtype=torch.int32, device=cuda)
    out = conv(req[:1] * 0, big, idx[:1], BLOCK_SIZE=64, NUM_TOPK_TOKENS=topk, BLOCK_STRIDE_ROWS=66)
    want = oracle.convert_req_index(np.zeros(1), big.cpu().numpy(), idx[:1].cpu().numpy(), 64, 66)
    assert np.array_equal(out.cpu().numpy(), want)


@pytest.mark.parametrize("splits", [1, 8, None])
@pytest.mark.parametrize("block_size,page_rows", [(64, 64), (64, 66), (2304, 2304)])
def test_paged_attention_equals_convert_then_attend(cuda, oracle, splits, block_size, page_rows):
    from sparse_utils import triton_convert_req_index_to_global_index as conv
    from titan_mla import triton_mla_sparse_attention, triton_mla_sparse_attention_paged
    from oracle import bf16_to_f32
    max_blocks = 4 if block_size == 2304 else 40
    num_blocks = 3 * max_blocks + 2
    log_case("paged attention", block_size, page_rows, splits)
    cache, rows, rows_np = paged_cache(cuda, num_blocks, block_size, page_rows, seed=31)
    bt = tables(cuda, 3, max_blocks, num_blocks, 7)
    g = W.gen(cuda, 32)
    T, topk = 6, 2176
    req = torch.tensor([2, 0, 1, 1, 2, 0], dtype=torch.int32, device=cuda)
    q = torch.randn(T, 16, 512, generator=g, device=cuda).to(torch.bfloat16)
    idx = torch.randint(0, max_blocks * block_size, (T, topk), generator=g, device=cuda, dtype=torch.int32)
    idx[1, -200:] = -1
    idx[2, :50] = max_blocks * block_size + 17          # beyond the table -> masked
    fused = triton_mla_sparse_attention_paged(q, cache, idx, req, bt, W.SM_SCALE, num_kv_splits=splits)
    flat_idx = conv(req, bt, idx, BLOCK_SIZE=block_size, NUM_TOPK_TOKENS=topk, BLOCK_STRIDE_ROWS=page_rows)
    two = triton_mla_sparse_attention(q, rows.view(-1, 1, 528), flat_idx.view(T, 1, topk), W.SM_SCALE,
                                      num_kv_splits=splits)
    torch.cuda.synchronize()
    assert torch.equal(fused, two)
    # against the oracle over each request's logically ordered cache
    btn, reqn, idxn = bt.cpu().numpy(), req.cpu().numpy(), idx.cpu().numpy()
    qn = q.view(torch.int16).cpu().numpy().view(np.uint16)
    got = fused.float().cpu().numpy()
    for t in range(T):
        logical = np.concatenate([rows_np[b * page_rows: b * page_rows + block_size] for b in btn[reqn[t]]])
        li = np.where((idxn[t] >= 0) & (idxn[t] < logical.shape[0]), idxn[t], -1)[None, :]
        want = bf16_to_f32(oracle.sparse_mla(qn[t:t + 1], logical, li, W.SM_SCALE, n_splits=1))[0]
        err = np.abs(got[t] - want)
        ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(want), 2.0 ** -126))) - 7)
        assert np.all(err <= np.maximum(MAX_ABS, ulp)) and err.mean() <= MEAN_ABS, (t, err.max())


def test_paged_attention_graph_and_bad_requests(cuda):
    from titan_mla import triton_mla_sparse_attention_paged
    cache, rows, _ = paged_cache(cuda, 40, 64, 66, seed=41)
    bt = tables(cuda, 2, 16, 40, 9)
    g = W.gen(cuda, 42)
    q = torch.randn(3, 16, 512, generator=g, device=cuda).to(torch.bfloat16)
    idx = torch.randint(0, 16 * 64, (3, 1, 2176), generator=g, device=cuda, dtype=torch.int32)
    req = torch.tensor([1, 5, 0], dtype=torch.int32, device=cuda)      # 5: no table row
    log_case("paged graph")
    ref = triton_mla_sparse_attention_paged(q, cache, idx, req, bt, W.SM_SCALE)
    torch.cuda.synchronize()
    assert torch.equal(ref[1], torch.zeros_like(ref[1]))              # every index masked -> 0
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = triton_mla_sparse_attention_paged(q, cache, idx, req, bt, W.SM_SCALE)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
