"""One decode step's sparse-attention chain end to end on the GPU, against the
oracle's functions applied one after the other:

  store_int8 of every context token's latent into a paged INT8 cache
  (kernels/titan_kv.py:7-28), the indexer's FP8 paged logits and top-512
  pools (integration/patch_decode_indexer.py:34-72), the pools' expansion
  with the context tail (integration/patch_indexer_sharding.py:92-99), the
  request-relative -> paged row mapping (integration/titan_backend.py:49-52)
  and the sparse MLA over the cache (kernels/titan_mla.py:452-581).

The GPU path is the library's own composition: titan_kv.store_int8,
sparse_indexer.indexer_decode_pool_topk and
titan_mla.triton_mla_sparse_attention_pooled (expansion, mapping and the
split kernel in one launch).  Bars: the cache bytes bit-exact; the pool
selection exact (the oracle selects on the GPU's logits, so rounding in the
logits cannot move the threshold; the logits themselves are checked in
test_gpu_indexer); the attention output within the MLA bar (mla_bar:
max-abs 2e-2 / mean-abs 2e-3, rare bf16 rounding flips of |ref| >= 2 up to
two ulps) of the oracle's reference reduction (one online-softmax stream,
BLOCK_N 32) over the rows the oracle's own expansion and mapping pick."""
import numpy as np
import pytest

import workloads as W
from conftest import log_case
from mla_bar import check_bar

pytestmark = pytest.mark.gpu

POOL = 4          # tokens per indexer pool
BLOCK = 64        # cache rows per page (MLA) and pools per page (indexer)
TOPK_POOLS = 512
TOPK = 2176       # index slots of the attention


@pytest.mark.parametrize("seq_lens,splits", [((9000, 6157, 12003), None), ((4100, 2051, 8190), 8),
                                              ((2050, 3, 5000), None)])
def test_decode_chain(cuda, oracle, seq_lens, splits):
    import torch
    from sparse_indexer import indexer_decode_pool_topk
    from titan_kv import store_int8
    from titan_mla import triton_mla_sparse_attention_pooled

    B = len(seq_lens)
    g = W.gen(cuda, 8100 + sum(seq_lens))
    rng = np.random.default_rng(sum(seq_lens))
    log_case("decode chain", seq_lens, splits)

    # MLA cache: each request's positions on its own random pages, written
    # through store_int8's slot mapping.
    max_blocks = (max(seq_lens) + BLOCK - 1) // BLOCK
    num_blocks = B * max_blocks + 3
    bt = rng.permutation(num_blocks)[: B * max_blocks].reshape(B, max_blocks).astype(np.int32)
    slots = np.concatenate([bt[r, np.arange(n) // BLOCK].astype(np.int64) * BLOCK + np.arange(n) % BLOCK
                            for r, n in enumerate(seq_lens)])
    x = (W.student_t3((slots.size, 512), g, cuda) * 0.5).to(torch.bfloat16)
    cache = torch.zeros(num_blocks, BLOCK, 528, dtype=torch.int8, device=cuda)
    store_int8(x, cache, torch.from_numpy(slots).to(cuda))
    torch.cuda.synchronize()
    cache_np = np.zeros((num_blocks, BLOCK, 528), dtype=np.uint8)
    oracle.store_int8(x.view(torch.int16).cpu().numpy().view(np.uint16), cache_np, slots)
    assert np.array_equal(cache.view(torch.uint8).cpu().numpy(), cache_np)
    cache_np = cache_np.reshape(-1, 528)

    # Indexer: complete pools of each request's context in random pages.
    pools_len = np.array([n // POOL for n in seq_lens], dtype=np.int32)
    per_req = (int(pools_len.max()) + BLOCK - 1) // BLOCK
    icache, nb = W.indexer_cache(cuda, g, B * per_req * BLOCK, BLOCK)
    ibt = torch.randperm(nb, generator=g, device=cuda).to(torch.int32)[: B * per_req].view(B, per_req).contiguous()
    qi = torch.randn(B, 1, W.INDEX_HEADS, 128, generator=g, device=cuda)
    qi = (qi * (448.0 / qi.abs().amax(dim=-1, keepdim=True))).to(torch.float8_e4m3fn)
    wi = (torch.randn(B, W.INDEX_HEADS, generator=g, device=cuda) * W.INDEX_HEADS ** -0.5).contiguous()
    lens = torch.from_numpy(pools_len).to(cuda)
    max_pools = per_req * BLOCK

    # GPU chain.
    q = torch.randn(B, 16, 512, generator=g, device=cuda).to(torch.bfloat16)
    req = torch.arange(B, dtype=torch.int32, device=cuda)
    seq = torch.tensor(seq_lens, dtype=torch.int32, device=cuda)
    bt_d = torch.from_numpy(bt).to(cuda)
    pools = indexer_decode_pool_topk(qi, icache, wi, lens, ibt, max_pools, k=TOPK_POOLS)
    out = triton_mla_sparse_attention_pooled(q, cache, pools, seq, POOL, req, bt_d, W.SM_SCALE, topk=TOPK,
                                             num_kv_splits=splits)
    torch.cuda.synchronize()

    # Oracle chain: the selection on the same logits, then expansion, mapping
    # and the reference attention.
    from sparse_indexer import fp8_paged_mqa_logits
    logits = fp8_paged_mqa_logits(qi, icache, wi, lens, ibt, max_pools, clean_logits=False)
    torch.cuda.synchronize()
    sel = oracle.indexer_topk(logits.cpu().numpy(), pools_len, TOPK_POOLS)
    pools_np = pools.cpu().numpy()
    assert np.array_equal(pools_np, sel)
    tokens = oracle.expand_pools(sel, np.array(seq_lens), POOL, out_cols=TOPK)
    rows = oracle.convert_req_index(np.arange(B), bt, tokens, BLOCK)
    for r, n in enumerate(seq_lens):   # every selected position is inside the request's context
        p = tokens[r][tokens[r] >= 0]
        assert p.size == min(n // POOL, TOPK_POOLS) * POOL + n % POOL and p.max() < n
    want = oracle.bf16_to_f32(oracle.sparse_mla(q.view(torch.int16).cpu().numpy().view(np.uint16), cache_np, rows,
                                                W.SM_SCALE, n_splits=1, groups=1, block_n=32))
    check_bar(out.float().cpu().numpy(), want, f"decode chain {seq_lens} splits={splits}")
