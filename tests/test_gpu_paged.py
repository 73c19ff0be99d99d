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
from mla_bar import check_bar

pytestmark = pytest.mark.gpu


def paged_cache(cuda, num_blocks, block_size, page_bytes, seed):
    """int8 [num_blocks, block_size, 528] cache whose pages start page_bytes
    apart (padding untouched), filled by store_int8 through its slot mapping;
    returns the cache and its rows as numpy [num_blocks, block_size, 528]."""
    from titan_kv import store_int8
    g = W.gen(cuda, seed)
    raw = torch.zeros(num_blocks * page_bytes, dtype=torch.int8, device=cuda)
    cache = torch.as_strided(raw, (num_blocks, block_size, 528), (page_bytes, 528, 1))
    n = num_blocks * block_size
    x = torch.randn(n, 512, generator=g, device=cuda).to(torch.bfloat16)
    store_int8(x, cache, torch.arange(n, device=cuda))
    torch.cuda.synchronize()
    return cache, cache.contiguous().view(torch.uint8).cpu().numpy()


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


def logical_attention(q, cache, idx, req, bt, splits, sm_scale):
    """Reference on the GPU: per token, its request's pages copied in
    block-table order into one contiguous cache, indexed by the raw
    positions, through the flat-index attention."""
    from titan_mla import triton_mla_sparse_attention
    outs = []
    for t in range(q.shape[0]):
        pages = cache[bt[int(req[t])].long()]                       # [max_blocks, block_size, 528]
        flat = pages.reshape(-1, 1, 528).contiguous()
        outs.append(triton_mla_sparse_attention(q[t:t + 1], flat, idx[t:t + 1].view(1, 1, -1), sm_scale,
                                                num_kv_splits=splits))
    return torch.cat(outs)


@pytest.mark.parametrize("splits", [1, 8, None])
@pytest.mark.parametrize("block_size,page_bytes", [(64, 64 * 528), (64, 66 * 528), (64, 36864), (2304, 2304 * 528)])
def test_paged_attention(cuda, oracle, splits, block_size, page_bytes):
    """Fused paged attention = per-token attention over the logically ordered
    cache (bit for bit), = convert + attend on the flat row view when the page
    stride is a whole number of rows (bit for bit), and within the attention
    bar of the oracle.  36864 bytes = 64 rows padded to a 4 KB multiple."""
    from sparse_utils import flat_kv_row_view, triton_convert_req_index_to_global_index as conv
    from titan_mla import triton_mla_sparse_attention, triton_mla_sparse_attention_paged
    from oracle import bf16_to_f32
    max_blocks = 4 if block_size == 2304 else 40
    num_blocks = 3 * max_blocks + 2
    log_case("paged attention", block_size, page_bytes, splits)
    cache, pages_np = paged_cache(cuda, num_blocks, block_size, page_bytes, seed=31)
    bt = tables(cuda, 3, max_blocks, num_blocks, 7)
    g = W.gen(cuda, 32)
    T, topk = 6, 2176
    req = torch.tensor([2, 0, 1, 1, 2, 0], dtype=torch.int32, device=cuda)
    q = torch.randn(T, 16, 512, generator=g, device=cuda).to(torch.bfloat16)
    idx = torch.randint(0, max_blocks * block_size, (T, topk), generator=g, device=cuda, dtype=torch.int32)
    idx[1, -200:] = -1
    idx[2, :50] = max_blocks * block_size + 17          # beyond the table -> masked
    if splits is None:   # the auto policy for this batch, pinned for the per-token references
        from titan_mla import _choose_num_kv_splits_mi355x
        splits = _choose_num_kv_splits_mi355x(T, 1, topk, torch.cuda.get_device_properties(0).multi_processor_count)
    fused = triton_mla_sparse_attention_paged(q, cache, idx, req, bt, W.SM_SCALE, num_kv_splits=splits)
    logical = logical_attention(q, cache, torch.where(idx < max_blocks * block_size, idx, -1), req, bt, splits,
                                W.SM_SCALE)
    torch.cuda.synchronize()
    assert torch.equal(fused, logical)
    if page_bytes % 528 == 0:
        rows, stride = flat_kv_row_view(cache, block_size)
        flat_idx = conv(req, bt, idx, BLOCK_SIZE=block_size, NUM_TOPK_TOKENS=topk, BLOCK_STRIDE_ROWS=stride)
        two = triton_mla_sparse_attention(q, rows.view(-1, 1, 528), flat_idx.view(T, 1, topk), W.SM_SCALE,
                                          num_kv_splits=splits)
        torch.cuda.synchronize()
        assert torch.equal(fused, two)
    # against the oracle over each request's logically ordered cache
    btn, reqn, idxn = bt.cpu().numpy(), req.cpu().numpy(), idx.cpu().numpy()
    qn = q.view(torch.int16).cpu().numpy().view(np.uint16)
    got = fused.float().cpu().numpy()
    for t in range(T):
        lc = pages_np[btn[reqn[t]]].reshape(-1, 528)
        li = np.where((idxn[t] >= 0) & (idxn[t] < lc.shape[0]), idxn[t], -1)[None, :]
        want = bf16_to_f32(oracle.sparse_mla(qn[t:t + 1], lc, li, W.SM_SCALE, n_splits=1))[0]
        check_bar(got[t], want, f"paged token {t}", max_ulp=1)   # this test's bar held one ulp before the shared bar


def test_paged_random_shapes(cuda):
    """Seeded random block sizes, page padding, request counts, table widths,
    request ids, positions (past the table, negative) and split counts: the
    fused paged attention equals per-token attention over the logically
    ordered cache bit for bit, and the flat path through the conversion when
    the page stride is a whole number of rows."""
    from sparse_utils import flat_kv_row_view, triton_convert_req_index_to_global_index as conv
    from titan_mla import triton_mla_sparse_attention, triton_mla_sparse_attention_paged
    rng = np.random.default_rng(515)
    g = W.gen(cuda, 515)
    for case in range(10):
        block_size = int(rng.choice([16, 48, 64, 200, 256, 1024]))
        pad_units = int(rng.choice([0, 0, 1, 7, 33]))          # extra 16-byte units per page
        page_bytes = block_size * 528 + 16 * pad_units
        reqs = int(rng.integers(1, 4))
        max_blocks = int(rng.integers(1, 12))
        num_blocks = reqs * max_blocks + int(rng.integers(0, 4))
        cache, _ = paged_cache(cuda, num_blocks, block_size, page_bytes, seed=600 + case)
        bt = tables(cuda, reqs, max_blocks, num_blocks, 700 + case)
        T = int(rng.integers(1, 6))
        topk = 32 * int(rng.integers(1, 70))
        splits = int(rng.choice([1, 2, 5, 8]))
        req = torch.from_numpy(rng.integers(0, reqs, size=T).astype(np.int32)).to(cuda)
        span = max_blocks * block_size
        idx = torch.from_numpy(rng.integers(-3, span + 50, size=(T, topk)).astype(np.int32)).to(cuda)
        log_case("paged random", case, block_size, pad_units, reqs, max_blocks, T, topk, splits)
        q = torch.randn(T, 16, 512, generator=g, device=cuda).to(torch.bfloat16)
        fused = triton_mla_sparse_attention_paged(q, cache, idx, req, bt, W.SM_SCALE, num_kv_splits=splits)
        logical = logical_attention(q, cache, torch.where(idx < span, idx, -1), req, bt, splits, W.SM_SCALE)
        torch.cuda.synchronize()
        assert torch.equal(fused, logical), case
        if page_bytes % 528 == 0:
            rows, stride = flat_kv_row_view(cache, block_size)
            flat_idx = conv(req, bt, idx, BLOCK_SIZE=block_size, NUM_TOPK_TOKENS=topk, BLOCK_STRIDE_ROWS=stride)
            two = triton_mla_sparse_attention(q, rows.view(-1, 1, 528), flat_idx.view(T, 1, topk), W.SM_SCALE,
                                              num_kv_splits=splits)
            torch.cuda.synchronize()
            assert torch.equal(fused, two), case


def test_paged_table_entries_outside_the_cache_are_masked(cuda):
    """A block-table entry that is not one of the cache's pages (negative or
    too large, e.g. a stale or unused slot) masks its positions."""
    from titan_mla import triton_mla_sparse_attention_paged
    cache, _ = paged_cache(cuda, 8, 64, 36864, seed=51)
    g = W.gen(cuda, 52)
    q = torch.randn(2, 16, 512, generator=g, device=cuda).to(torch.bfloat16)
    bt = torch.tensor([[3, -1, 1, 8], [2, 5, 100000, 0]], dtype=torch.int32, device=cuda)
    req = torch.tensor([0, 1], dtype=torch.int32, device=cuda)
    idx = torch.randint(0, 4 * 64, (2, 2176), generator=g, device=cuda, dtype=torch.int32)
    log_case("paged bad table entries")
    out = triton_mla_sparse_attention_paged(q, cache, idx, req, bt, W.SM_SCALE, num_kv_splits=4)
    bad = ((idx // 64 == 1) | (idx // 64 == 3)) & (req[:, None] == 0) | (idx // 64 == 2) & (req[:, None] == 1)
    clean = torch.where(bad, torch.full_like(idx, -1), idx)
    good_bt = torch.where(bt < 0, 0, torch.where(bt >= 8, 0, bt))
    ref = triton_mla_sparse_attention_paged(q, cache, clean, req, good_bt, W.SM_SCALE, num_kv_splits=4)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def test_paged_attention_graph_and_bad_requests(cuda):
    from titan_mla import triton_mla_sparse_attention_paged
    cache, _ = paged_cache(cuda, 40, 64, 66 * 528, seed=41)
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


@pytest.mark.parametrize("pool_size,with_tail,dtype", [(4, True, torch.int32), (4, False, torch.int64),
                                                       (1, True, torch.int32), (5, True, torch.int64)])
def test_expand_pools_matches_oracle(cuda, oracle, pool_size, with_tail, dtype):
    from sparse_utils import expand_pools_and_append_tail, expand_pools_to_tokens
    log_case("expand pools", pool_size, with_tail, dtype)
    g = W.gen(cuda, 61)
    rows, k = 7, 512
    pools = torch.randint(-3, 20000, (rows, k), generator=g, device=cuda).to(dtype)
    if dtype == torch.int64:
        pools[0, :5] = 1 << 33                      # not an int32 pool id -> -1
    lens = torch.randint(0, 90000, (rows,), generator=g, device=cuda, dtype=torch.int32)
    if with_tail:
        got = expand_pools_and_append_tail(pools, lens, pool_size)
        want = oracle.expand_pools(np.where(pools.cpu().numpy() > 2 ** 31 - 1, -1, pools.cpu().numpy()),
                                   lens.cpu().numpy(), pool_size)
    else:
        valid = pools >= 0
        valid[1, 7] = False
        got = expand_pools_to_tokens(pools, valid, k * pool_size, pool_size)
        pn = np.where(valid.cpu().numpy(), pools.cpu().numpy(), -1)
        want = oracle.expand_pools(np.where(pn > 2 ** 31 - 1, -1, pn), None, pool_size)
    torch.cuda.synchronize()
    assert got.shape == want.shape and np.array_equal(got.cpu().numpy(), want)


def test_expand_and_convert_random_shapes(cuda, oracle):
    """Seeded random pool counts, pool sizes, lengths and id widths for the
    expansion, and random block sizes, page rows, tables and positions for the
    conversion, each bit-exact against the oracle."""
    from sparse_utils import expand_pools_and_append_tail, triton_convert_req_index_to_global_index as conv
    rng = np.random.default_rng(8181)
    for case in range(12):
        rows, k = int(rng.integers(1, 9)), int(rng.integers(1, 700))
        pool_size = int(rng.integers(1, 9))
        dtype = np.int64 if case % 2 else np.int32
        pools = rng.integers(-5, 40000, size=(rows, k)).astype(dtype)
        lens = rng.integers(-3, 200000, size=rows).astype(np.int32)
        log_case("expand random", case, rows, k, pool_size, dtype.__name__)
        got = expand_pools_and_append_tail(torch.from_numpy(pools).to(cuda), torch.from_numpy(lens).to(cuda),
                                           pool_size)
        torch.cuda.synchronize()
        assert np.array_equal(got.cpu().numpy(), oracle.expand_pools(pools, lens, pool_size)), case
    for case in range(12):
        block_size = int(rng.choice([1, 16, 64, 100, 256, 2304]))
        page_rows = block_size + int(rng.choice([0, 0, 1, 3]))
        reqs, max_blocks = int(rng.integers(1, 5)), int(rng.integers(1, 30))
        bt = rng.integers(-2, 5000, size=(reqs, max_blocks)).astype(np.int32)
        T, topk = int(rng.integers(1, 10)), 32 * int(rng.integers(1, 70))
        req = rng.integers(-1, reqs + 1, size=T).astype(np.int32)
        span = max_blocks * block_size
        idx = rng.integers(-4, span + 40, size=(T, topk)).astype(np.int32)
        log_case("convert random", case, block_size, page_rows, reqs, max_blocks, T, topk)
        got = conv(torch.from_numpy(req).to(cuda), torch.from_numpy(bt).to(cuda), torch.from_numpy(idx).to(cuda),
                   BLOCK_SIZE=block_size, NUM_TOPK_TOKENS=topk, BLOCK_STRIDE_ROWS=page_rows)
        torch.cuda.synchronize()
        assert np.array_equal(got.cpu().numpy(), oracle.convert_req_index(req, bt, idx, block_size, page_rows)), case


@pytest.mark.parametrize("splits", [1, 8, None])
@pytest.mark.parametrize("with_tail", [True, False])
def test_pooled_attention_equals_expand_then_paged(cuda, splits, with_tail):
    """Pool ids straight to attention = expansion into a -1-filled 2176-slot
    buffer, then the paged attention (bit for bit)."""
    from sparse_utils import expand_pools_and_append_tail, expand_pools_to_tokens
    from titan_mla import triton_mla_sparse_attention_paged, triton_mla_sparse_attention_pooled
    log_case("pooled attention", splits, with_tail)
    block_size, max_blocks = 64, 40
    cache, _ = paged_cache(cuda, 3 * max_blocks + 2, block_size, 36864, seed=71)
    bt = tables(cuda, 3, max_blocks, 3 * max_blocks + 2, 17)
    g = W.gen(cuda, 72)
    T, pool_size, k = 5, 4, 512
    ctx = max_blocks * block_size
    req = torch.tensor([0, 2, 1, 0, 2], dtype=torch.int32, device=cuda)
    q = torch.randn(T, 16, 512, generator=g, device=cuda).to(torch.bfloat16)
    pools = torch.randint(-1, ctx // pool_size, (T, k), generator=g, device=cuda, dtype=torch.int32)
    lens = torch.randint(ctx - 50, ctx, (T,), generator=g, device=cuda, dtype=torch.int32)
    seq = lens if with_tail else None
    fused = triton_mla_sparse_attention_pooled(q, cache, pools, seq, pool_size, req, bt, W.SM_SCALE, topk=2176,
                                               num_kv_splits=splits)
    exp = (expand_pools_and_append_tail(pools, lens, pool_size) if with_tail
           else expand_pools_to_tokens(pools, pools >= 0, k * pool_size, pool_size))
    buf = torch.full((T, 2176), -1, dtype=torch.int32, device=cuda)
    buf[:, : exp.shape[1]] = exp
    two = triton_mla_sparse_attention_paged(q, cache, buf, req, bt, W.SM_SCALE, num_kv_splits=splits)
    torch.cuda.synchronize()
    assert torch.equal(fused, two)


@pytest.mark.parametrize("max_blocks", [8000, 9000])
def test_paged_long_block_tables(cuda, max_blocks):
    """Block-table rows up to 8192 entries are staged in LDS, longer ones are
    read from memory; both give the logical-cache result."""
    log_case("paged long table", max_blocks)
    block_size = 1
    num_blocks = max_blocks + 5
    cache, _ = paged_cache(cuda, num_blocks, block_size, 528, seed=81)
    bt = tables(cuda, 1, max_blocks, num_blocks, 19)
    g = W.gen(cuda, 82)
    q = torch.randn(2, 16, 512, generator=g, device=cuda).to(torch.bfloat16)
    req = torch.zeros(2, dtype=torch.int32, device=cuda)
    idx = torch.randint(0, max_blocks, (2, 2176), generator=g, device=cuda, dtype=torch.int32)
    from titan_mla import triton_mla_sparse_attention_paged
    fused = triton_mla_sparse_attention_paged(q, cache, idx, req, bt, W.SM_SCALE, num_kv_splits=8)
    ref = logical_attention(q, cache, idx, req, bt, 8, W.SM_SCALE)
    torch.cuda.synchronize()
    assert torch.equal(fused, ref)
