"""GPU parity of the sparse indexer decode scoring: FP8 paged MQA logits and
the top-k pool selection, against the oracle.

Tolerances.  Logits: the fp8 products are exact in fp32; the kernel sums 128
of them per head on the matrix cores and the heads in fp32 in another order
than the oracle's float64, so |d| <= 2^-15 * sum_h |w_h s_j| sum_d |q k|
(a bound on fp32 accumulation error for these lengths, with margin).
Selection: integer positions, compared exactly -- against the oracle's
selection on the same (GPU) logits, so rounding differences in the logits
cannot move the threshold."""
import numpy as np
import pytest

import workloads as W
from conftest import log_case

pytestmark = pytest.mark.gpu


def host(t):
    import torch
    if t.dtype == torch.float8_e4m3fn:
        t = t.view(torch.uint8)
    return t.cpu().numpy()


def pages_of(cache):
    """[num_blocks, page_bytes] uint8 view of a (possibly padded) fused cache."""
    import torch
    nb = cache.shape[0]
    page = cache.stride(0)
    flat = torch.as_strided(cache, (nb, page), (page, 1))
    return flat.cpu().numpy()


def check_logits(oracle, got, q, cache, w, lens, bt, max_len, clean, rows=None):
    T = got.shape[0]
    rows = range(T) if rows is None else rows
    qn = host(q).reshape(T, q.shape[-2], q.shape[-1])
    want, mag = oracle.fp8_paged_mqa_logits(qn, pages_of(cache), cache.shape[1], host(w), host(lens), host(bt),
                                            max_len, clean=clean, bound=True)
    g = got.cpu().numpy().astype(np.float64)
    for t in rows:
        n = int(min(max(int(lens[t]), 0), bt.shape[1] * cache.shape[1], max_len))
        fin = np.isfinite(want[t, :n])
        assert np.array_equal(np.isneginf(g[t, :n]), np.isneginf(want[t, :n])), f"row {t}: masked positions differ"
        err = np.abs(g[t, :n][fin] - want[t, :n][fin])
        bound = 2.0 ** -15 * mag[t, :n][fin] + 1e-30
        assert (err <= bound).all(), f"row {t}: max err {err.max():.3e} (ratio {(err / bound).max():.2f})"
        if clean:
            assert np.all(np.isneginf(g[t, n:max_len]))


@pytest.mark.parametrize("heads", [16, 32, 48, 64])
def test_logits_small(cuda, oracle, heads):
    import torch
    from sparse_indexer import fp8_paged_mqa_logits
    g = torch.Generator(device=cuda).manual_seed(100 + heads)
    T, bs = 3, 64
    cache, nb = W.indexer_cache(cuda, g, 3 * 1500, bs, page_pad=48)
    perm = torch.randperm(nb, generator=g, device=cuda).to(torch.int32)
    bt = perm[: T * (nb // T)].view(T, nb // T).contiguous()
    bt[0, 2] = nb + 3                 # outside the cache: that page's keys are -inf
    bt[2, 0] = -1
    qf = torch.randn(T, 1, heads, 128, generator=g, device=cuda)
    q = (qf * (448.0 / qf.abs().amax(dim=-1, keepdim=True))).to(torch.float8_e4m3fn)
    w = torch.randn(T, heads, generator=g, device=cuda) / heads ** 0.5
    lens = torch.tensor([1500, 777, 1], dtype=torch.int32, device=cuda)
    max_len = 1600
    for clean in (True, False):
        log_case("indexer logits", heads, "clean", clean)
        got = fp8_paged_mqa_logits(q, cache, w, lens, bt, max_len, clean_logits=clean)
        torch.cuda.synchronize()
        check_logits(oracle, got, q, cache, w, lens, bt, max_len, clean)


def test_logits_block_sizes_and_mtp(cuda, oracle):
    """Block sizes that split 16-key groups across pages, and next_n = 2
    (each query row sees its own causal length)."""
    import torch
    from sparse_indexer import fp8_paged_mqa_logits
    g = torch.Generator(device=cuda).manual_seed(7)
    for bs in (8, 24, 100):
        cache, nb = W.indexer_cache(cuda, g, 2 * 600, bs)
        bt = torch.randperm(nb, generator=g, device=cuda).to(torch.int32)[: 2 * (nb // 2)].view(2, -1).contiguous()
        bt[0, 2] = -1     # a group whose first keys sit on this page and the rest on the next (valid) one
        q = (torch.randn(2, 2, 32, 128, generator=g, device=cuda) * 100).to(torch.float8_e4m3fn)
        w = torch.randn(4, 32, generator=g, device=cuda) / 32 ** 0.5
        lens = torch.tensor([599, 313], dtype=torch.int32, device=cuda)
        log_case("indexer logits block", bs, "next_n 2")
        got = fp8_paged_mqa_logits(q, cache, w, lens, bt, 640)
        torch.cuda.synchronize()
        rows_ctx = torch.tensor([598, 599, 312, 313], dtype=torch.int32)
        check_logits(oracle, got, q.view(4, 1, 32, 128), cache, w, rows_ctx, bt.repeat_interleave(2, 0), 640, True)


@pytest.fixture(scope="module")
def decode_b8(cuda):
    import torch
    g = torch.Generator(device=cuda).manual_seed(W.SEED_FIXTURE)
    log_case("indexer decode B=8 inputs (262144-token context, 65536 pools per request)")
    return W.indexer_decode_inputs(cuda, g)


def test_logits_full_context(cuda, oracle, decode_b8):
    import torch
    from sparse_indexer import fp8_paged_mqa_logits
    q, cache, w, lens, bt, pools = decode_b8
    log_case("indexer logits B=8 x 65536 pools")
    got = fp8_paged_mqa_logits(q, cache, w, lens, bt, pools)
    torch.cuda.synchronize()
    check_logits(oracle, got, q, cache, w, lens, bt, pools, True, rows=[0, 5])


def test_topk_matches_oracle(cuda, oracle, decode_b8):
    import torch
    from sparse_indexer import fp8_paged_mqa_logits, indexer_topk, indexer_decode_pool_topk
    q, cache, w, lens, bt, pools = decode_b8
    logits = fp8_paged_mqa_logits(q, cache, w, lens, bt, pools, clean_logits=False)
    log_case("indexer top-512 B=8")
    got = indexer_topk(logits, lens, 512)
    torch.cuda.synchronize()
    want = oracle.indexer_topk(logits.cpu().numpy(), lens.cpu().numpy(), 512)
    assert np.array_equal(got.cpu().numpy(), want)
    fused = indexer_decode_pool_topk(q, cache, w, lens, bt, pools)
    torch.cuda.synchronize()
    assert torch.equal(fused, got)


def test_topk_ties_specials_and_short_rows(cuda, oracle):
    import torch
    from sparse_indexer import indexer_topk
    g = torch.Generator(device=cuda).manual_seed(11)
    rows, n = 6, 70000
    x = torch.randn(rows, n, generator=g, device=cuda)
    x[1] = torch.randint(0, 7, (n,), generator=g, device=cuda).float()          # heavy ties
    x[2, ::3] = float("nan")
    x[2, 1::7] = float("-inf")
    x[2, 5::11] = float("inf")
    x[3] = 0.0                                                                   # all equal
    x[4, :] = -torch.arange(n, device=cuda, dtype=torch.float32)                  # sorted descending
    lens = torch.tensor([n, n, 65536, 40000, 512, 100], dtype=torch.int32, device=cuda)
    for k in (512, 1, 2048):
        log_case("indexer top-k special rows", k)
        got = indexer_topk(x, lens, k)
        torch.cuda.synchronize()
        want = oracle.indexer_topk(x.cpu().numpy(), lens.cpu().numpy(), k)
        assert np.array_equal(got.cpu().numpy(), want), k


@pytest.mark.parametrize("copies", [1, 4])
@pytest.mark.parametrize("n,k", [
    (4096, 512),      # one workgroup over the row, 4 keys per thread
    (32768, 16384),   # one workgroup over the row, 32 keys per thread (chunks would not exceed k)
    (16384, 512),     # 512-thread workgroups over chunks of 4096, 2048 candidates
    (65536, 512),     # 1024-thread workgroups over chunks of 8192, 4096 candidates (from 32 rows:
                      # 512-thread workgroups over the same chunks)
    (20000, 8192),    # chunks of 16384, 16384 candidates
    (140000, 4096),   # too many candidates: sweeps over the row
])
def test_topk_every_plan(cuda, oracle, n, k, copies):
    """Each execution plan of the top-k, with ragged, clamped, tied and NaN
    rows; chunk boundaries at 4096, 8192 and 16384 positions.  copies = 4
    repeats the row set (40 rows), which takes the throughput plan (8192-
    position chunks) where it applies."""
    import torch
    from sparse_indexer import indexer_topk
    g = torch.Generator(device=cuda).manual_seed(n + k + copies)
    lens_list = [n, n - 1, min(n, 4097), min(n, 8193), min(n, 16385), k + 1, k, 3, -5, n + 1000] * copies
    rows = len(lens_list)
    x = torch.randn(rows, n, generator=g, device=cuda)
    x[1] = torch.randint(0, 3, (n,), generator=g, device=cuda).float()     # heavy ties
    x[2, ::2] = float("nan")
    x[3] = 1.0                                                              # all equal
    x[4, :] = torch.arange(n, device=cuda, dtype=torch.float32)             # ascending: the tail wins
    lens = torch.tensor(lens_list, dtype=torch.int32, device=cuda)
    log_case("indexer top-k plan", n, k)
    got = indexer_topk(x, lens, k)
    torch.cuda.synchronize()
    want = oracle.indexer_topk(x.cpu().numpy(), np.clip(lens.cpu().numpy(), 0, n), k)
    assert np.array_equal(got.cpu().numpy(), want)


@pytest.mark.parametrize("n,k", [(4095, 512), (70001, 512)])
def test_topk_unaligned_rows(cuda, oracle, n, k):
    """Row strides that are not a multiple of 4 floats (pool counts of any
    size): keys load one at a time; one workgroup per row and the two stages."""
    import torch
    from sparse_indexer import indexer_topk
    g = torch.Generator(device=cuda).manual_seed(n)
    x = torch.randn(3, n, generator=g, device=cuda)
    x[1] = torch.randint(0, 5, (n,), generator=g, device=cuda).float()
    lens = torch.tensor([n, n - 7, k + 3], dtype=torch.int32, device=cuda)
    log_case("indexer top-k unaligned rows", n, k)
    got = indexer_topk(x, lens, k)
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy(), oracle.indexer_topk(x.cpu().numpy(), lens.cpu().numpy(), k))


def test_decode_pool_topk_mtp_and_table_capacity(cuda, oracle):
    """The fused decode call with next_n = 2 (each query row its own causal
    length) and a context longer than its block table holds (the positions
    the table cannot hold are neither scored nor selected)."""
    import torch
    from sparse_indexer import fp8_paged_mqa_logits, indexer_decode_pool_topk
    g = torch.Generator(device=cuda).manual_seed(21)
    bs, per_req = 64, 40
    cache, nb = W.indexer_cache(cuda, g, 3 * per_req * bs, bs)
    bt = torch.randperm(nb, generator=g, device=cuda).to(torch.int32)[: 3 * per_req].view(3, per_req).contiguous()
    q = (torch.randn(3, 2, 32, 128, generator=g, device=cuda) * 60).to(torch.float8_e4m3fn)
    w = torch.randn(6, 32, generator=g, device=cuda) / 32 ** 0.5
    ctx = torch.tensor([per_req * bs, 700, per_req * bs + 500], dtype=torch.int32, device=cuda)
    max_pools = per_req * bs + 512
    log_case("indexer decode pool top-k, next_n 2, context past the table")
    got = indexer_decode_pool_topk(q, cache, w, ctx, bt, max_pools)
    logits = fp8_paged_mqa_logits(q, cache, w, ctx, bt, max_pools, clean_logits=False)
    torch.cuda.synchronize()
    rows_ctx = np.array([per_req * bs - 1, per_req * bs, 699, 700, per_req * bs, per_req * bs])   # clamped to the table
    want = oracle.indexer_topk(logits.cpu().numpy(), rows_ctx, 512)
    assert np.array_equal(got.cpu().numpy(), want)
    # the logits of those rows against the float64 oracle (scored positions only)
    check_logits(oracle, logits, q.view(6, 1, 32, 128), cache, w, torch.from_numpy(rows_ctx),
                 bt.repeat_interleave(2, 0), max_pools, False)
    # next_n = 1 (the decode case): the same clamp, applied by narrowing the columns
    q1, w1 = q[:, 1:].contiguous(), w.view(3, 2, 32)[:, 1].contiguous()
    got1 = indexer_decode_pool_topk(q1, cache, w1, ctx, bt, max_pools)
    logits1 = fp8_paged_mqa_logits(q1, cache, w1, ctx, bt, max_pools, clean_logits=False)
    torch.cuda.synchronize()
    ctx1 = np.minimum(ctx.cpu().numpy(), per_req * bs)
    assert np.array_equal(got1.cpu().numpy(), oracle.indexer_topk(logits1.cpu().numpy(), ctx1, 512))


def test_logits_nan_codes(cuda, oracle):
    """E4M3 NaN codes in keys and in one head's query: the NaN products are
    dropped by the relu (fmax), as the oracle defines."""
    import torch
    from sparse_indexer import fp8_paged_mqa_logits, indexer_topk
    g = torch.Generator(device=cuda).manual_seed(31)
    bs = 64
    cache, nb = W.indexer_cache(cuda, g, 2 * 1024, bs)
    bt = torch.arange(nb, device=cuda, dtype=torch.int32).view(2, -1).contiguous()
    pages = torch.as_strided(cache, (nb, cache.stride(0)), (cache.stride(0), 1))   # page bytes
    pages[0, 5 * 128 + 17] = 0x7F      # key 5 of row 0 (page 0), dim 17
    pages[3, 0] = 0xFF                 # key 192 of row 0, dim 0
    pages[nb - 1, 63 * 128 + 127] = 0x7F                                   # the last key of row 1, dim 127
    pages[nb - 1, 64 * 128 + 4 * 62: 64 * 128 + 4 * 63] = torch.tensor(    # key 1022 of row 1: NaN scale
        [0x00, 0x00, 0xC0, 0x7F], dtype=torch.uint8, device=cuda)
    qf = torch.randn(2, 1, 32, 128, generator=g, device=cuda)
    q = (qf * (448.0 / qf.abs().amax(dim=-1, keepdim=True))).to(torch.float8_e4m3fn)
    q.view(torch.uint8)[1, 0, 9, 40] = 0x7F   # head 9 of row 1
    w = torch.randn(2, 32, generator=g, device=cuda) / 32 ** 0.5
    lens = torch.tensor([1024, 1024], dtype=torch.int32, device=cuda)
    log_case("indexer logits with NaN codes")
    got = fp8_paged_mqa_logits(q, cache, w, lens, bt, 1024)
    torch.cuda.synchronize()
    check_logits(oracle, got, q, cache, w, lens, bt, 1024, True)
    g0 = got.cpu()
    assert g0[0, 5] == 0 and g0[0, 192] == 0 and g0[1, 1022] == 0 and g0[1, 1023] == 0
    assert torch.isfinite(g0).all()
    top = indexer_topk(got, lens, 512)
    torch.cuda.synchronize()
    assert np.array_equal(top.cpu().numpy(), oracle.indexer_topk(g0.numpy(), lens.cpu().numpy(), 512))


def test_logits_negative_and_zero_scales(cuda, oracle):
    """Keys with negative, -0.0 and +0.0 scales (the writer only makes
    positive ones): relu(s q.k) for s < 0 keeps the keys whose product is
    negative, which the kernels get by flipping the key's E4M3 sign bits and
    scaling by |s|; zero scales give 0.  Both logits kernels (per-token rows
    and rows sharing one table) against the oracle, and bit-identical to
    each other."""
    import torch
    from sparse_indexer import fp8_paged_mqa_logits
    g = torch.Generator(device=cuda).manual_seed(41)
    bs, pools, T = 64, 1536, 20
    cache, nb = W.indexer_cache(cuda, g, pools, bs)
    pages = torch.as_strided(cache, (nb, cache.stride(0)), (cache.stride(0), 1))
    sc = pages[:, bs * 128: bs * 132].contiguous().view(torch.float32)        # [nb, bs] scales
    flip = torch.rand(sc.shape, generator=g, device=cuda) < 0.3
    sc = torch.where(flip, -sc, sc)
    sc[0, 3], sc[1, 7], sc[2, 0] = -0.0, 0.0, -sc[2, 0].abs()
    pages[:, bs * 128: bs * 132] = sc.view(torch.uint8)
    qf = torch.randn(T, 1, 32, 128, generator=g, device=cuda)
    q = (qf * (448.0 / qf.abs().amax(dim=-1, keepdim=True))).to(torch.float8_e4m3fn)
    w = (torch.randn(T, 32, generator=g, device=cuda) / 32 ** 0.5).contiguous()
    lens = torch.randint(pools // 2, pools + 1, (T,), generator=g, device=cuda, dtype=torch.int32)
    table = torch.arange(nb, device=cuda, dtype=torch.int32)
    shared = table[None, :].expand(T, nb)
    log_case("indexer logits with negative and zero scales")
    got = fp8_paged_mqa_logits(q, cache, w, lens, shared, pools)
    per_row = fp8_paged_mqa_logits(q, cache, w, lens, shared.contiguous(), pools)
    torch.cuda.synchronize()
    assert torch.equal(got, per_row)
    check_logits(oracle, got, q, cache, w, lens, shared.contiguous(), pools, True)
    assert got[:, 3].eq(0).all() and got[:, 64 + 7].eq(0).all()


def test_logits_random_shapes(cuda, oracle):
    """Seeded random batch, next_n, heads, block sizes (straddling and not),
    page padding, contexts, table entries outside the cache, clean or not."""
    import torch
    from sparse_indexer import fp8_paged_mqa_logits
    rng = np.random.default_rng(77)
    g = torch.Generator(device=cuda).manual_seed(77)
    for case in range(10):
        B, next_n = int(rng.integers(1, 5)), int(rng.choice([1, 2]))
        H = int(rng.choice([16, 32, 48, 64]))
        bs = int(rng.choice([8, 16, 24, 64, 100, 128]))
        per_req = int(rng.integers(1, 6000 // bs + 2))
        cache, nb = W.indexer_cache(cuda, g, B * per_req * bs, bs, page_pad=int(rng.choice([0, 48])))
        bt = torch.randperm(nb, generator=g, device=cuda).to(torch.int32)[: B * per_req].view(B, per_req).contiguous()
        for r in range(B):
            if rng.random() < 0.4:
                bt[r, int(rng.integers(0, per_req))] = int(rng.choice([-1, nb, nb + 7]))
        q = (torch.randn(B, next_n, H, 128, generator=g, device=cuda) * 80).to(torch.float8_e4m3fn)
        w = torch.randn(B * next_n, H, generator=g, device=cuda) / H ** 0.5
        ctx = torch.from_numpy(rng.integers(0, per_req * bs + 40, size=B).astype(np.int32)).to(cuda)
        max_len = per_req * bs + int(rng.integers(0, 70))
        clean = bool(rng.random() < 0.5)
        log_case("indexer logits random", case, B, next_n, H, bs, per_req, max_len, clean)
        got = fp8_paged_mqa_logits(q, cache, w, ctx, bt, max_len, clean_logits=clean)
        torch.cuda.synchronize()
        offs = np.arange(next_n) - (next_n - 1)
        rows_ctx = (ctx.cpu().numpy()[:, None] + offs[None, :]).reshape(-1)
        check_logits(oracle, got, q.view(B * next_n, 1, H, 128), cache, w, torch.from_numpy(rows_ctx),
                     bt.repeat_interleave(next_n, 0), max_len, clean)


def test_topk_random_shapes(cuda, oracle):
    """Seeded random row counts, row lengths, k and lengths (every plan
    appears), each against the oracle's selection."""
    import torch
    from sparse_indexer import indexer_topk
    rng = np.random.default_rng(2026)
    g = torch.Generator(device=cuda).manual_seed(2026)
    for case in range(24):
        n = int(rng.choice([rng.integers(1, 5000), rng.integers(5000, 40000), rng.integers(40000, 150000)]))
        k = int(rng.integers(1, min(n, 20000) + 1))
        rows = int(rng.integers(1, 5))
        x = torch.randn(rows, n, generator=g, device=cuda)
        if case % 3 == 1:
            x = torch.round(x * 2)                      # many ties
        lens = torch.from_numpy(rng.integers(-2, n + 3, size=rows).astype(np.int32)).to(cuda)
        log_case("indexer top-k random", case, rows, n, k)
        got = indexer_topk(x, lens, k)
        torch.cuda.synchronize()
        want = oracle.indexer_topk(x.cpu().numpy(), lens.cpu().numpy(), k)
        assert np.array_equal(got.cpu().numpy(), want), (case, rows, n, k)


def test_decode_graph_replay(cuda, decode_b8):
    import torch
    from sparse_indexer import indexer_decode_pool_topk
    q, cache, w, lens, bt, pools = decode_b8
    fn = lambda: indexer_decode_pool_topk(q, cache, w, lens, bt, pools)
    log_case("indexer decode graph replay")
    eager = fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = fn()
    for i in range(3):
        captured.fill_(-7)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, eager), i
        fn()
        torch.cuda.synchronize()


@pytest.mark.slow
def test_prefill_shape_sampled_rows(cuda, oracle):
    """The reference's prefill indexer shape: 2048 query rows of one request
    at the end of a 262144-token context, each scoring the complete pools
    before it (65024..65536 of 65536), then its top 512.  Logits of sampled
    rows against the float64 oracle; the selection of every row bit-exact
    against the oracle's selection on the same GPU logits."""
    import torch
    from sparse_indexer import fp8_paged_mqa_logits, indexer_topk
    g = torch.Generator(device=cuda).manual_seed(2048)
    q, cache, w, lens, bt, pools = W.indexer_prefill_inputs(cuda, g)
    log_case("indexer prefill shape: 2048 rows x 65536 pools")
    logits = fp8_paged_mqa_logits(q, cache, w, lens, bt, pools, clean_logits=False)
    top = indexer_topk(logits, lens, 512)
    torch.cuda.synchronize()
    rows = [0, 1, 777, 2046, 2047]
    sel = torch.as_tensor(rows, device=cuda)
    check_logits(oracle, logits.index_select(0, sel), q.view(torch.uint8).index_select(0, sel), cache, w.index_select(0, sel),
                 lens.index_select(0, sel), bt.index_select(0, sel), pools, clean=False)
    want = oracle.indexer_topk(logits.cpu().numpy(), lens.cpu().numpy(), 512)
    assert np.array_equal(top.cpu().numpy(), want)


@pytest.mark.parametrize("heads", [16, 32, 64])
def test_shared_table_rows_kernel(cuda, oracle, heads):
    """Rows sharing one block table (row stride 0: a request's prefill
    chunk) take the row-tiled logits kernel: bit-identical to the per-token
    kernel on the same table materialised per row, and against the oracle;
    37 rows (not a multiple of the 16-row block) with lengths 0, short, odd,
    past the table, and the full context, a padded page stride and one table
    entry outside the cache, clean and not."""
    import torch
    from sparse_indexer import fp8_paged_mqa_logits
    g = torch.Generator(device=cuda).manual_seed(300 + heads)
    bs, pools = 64, 2500
    cache, nb = W.indexer_cache(cuda, g, pools + 200, bs, page_pad=32)
    per_req = (pools + bs - 1) // bs
    table = torch.randperm(nb, generator=g, device=cuda).to(torch.int32)[:per_req]
    table[5] = nb + 3                                   # outside the cache: its keys are -inf
    T = 37
    lens = torch.randint(0, pools + 1, (T,), generator=g, device=cuda, dtype=torch.int32)
    lens[:6] = torch.tensor([0, 1, 17, pools, pools + 500, 1000], dtype=torch.int32, device=cuda)
    qf = torch.randn(T, 1, heads, 128, generator=g, device=cuda)
    q = (qf * (448.0 / qf.abs().amax(dim=-1, keepdim=True))).to(torch.float8_e4m3fn)
    w = (torch.randn(T, heads, generator=g, device=cuda) * heads ** -0.5).contiguous()
    shared = table[None, :].expand(T, per_req)
    for clean in (True, False):
        log_case("indexer shared-table rows", heads, clean)
        got = fp8_paged_mqa_logits(q, cache, w, lens, shared, pools, clean_logits=clean)
        ref = fp8_paged_mqa_logits(q, cache, w, lens, shared.contiguous(), pools, clean_logits=clean)
        torch.cuda.synchronize()
        if clean:
            assert torch.equal(got, ref)
        else:   # unwritten positions hold whatever torch.empty gave: compare the written ones
            n = torch.arange(pools, device=cuda)[None, :] < lens.clamp(max=pools)[:, None].long()
            assert torch.equal(got[n], ref[n])
        check_logits(oracle, got, q, cache, w, lens, shared.contiguous(), pools, clean, rows=range(0, T, 6))
