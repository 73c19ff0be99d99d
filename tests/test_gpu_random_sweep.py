"""Seeded random sweeps over the entry points, each case against the oracle:
sparse MLA over flat rows (1-33 tokens, 1-40 heads, top-k 32-2848, split
counts auto / forced 1-99, masked and out-of-range indices, latents of
magnitude 0.01, 1 and 30 with the attention bar scaled by that magnitude:
the 2e-2 bar is stated for O(1) latents, and the bf16(p * scale) operand's
rounding moves an output by a fixed fraction of the rows' magnitude), the
top-k selection (1-33 rows, 1-140000 positions, ties, NaN and -inf keys,
lengths past both ends), the MoE aligner (every batch size, invalid ids,
int32 and int64) and the writer (strided rows, scattered int32 / int64 slots
with skipped -1 entries).  The integer paths are bit-exact."""
import numpy as np
import pytest
import torch

import workloads as W
from conftest import log_case
from mla_bar import check_bar

pytestmark = pytest.mark.gpu

CASES = 60


def u16(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.fixture(scope="module")
def caches(cuda):
    from titan_kv import store_int8
    g = W.gen(cuda, 8100)
    out = {}
    for n, scale in ((300, 1.0), (7000, 1.0), (70000, 1.0), (7001, 30.0), (301, 0.01)):
        x = (torch.randn(n, 512, generator=g, device=cuda) * scale).to(torch.bfloat16)
        cache = torch.zeros(-(-n // 256), 256, 528, dtype=torch.int8, device=cuda)
        store_int8(x, cache, torch.arange(n, device=cuda))
        rows = cache.contiguous().view(torch.uint8).cpu().numpy().reshape(-1, 528)[:n]
        out[n] = (cache.view(-1, 1, 528)[:n], rows, scale)
    torch.cuda.synchronize()
    return out


def test_sparse_mla_random(cuda, oracle, caches):
    from oracle import bf16_to_f32
    from test_gpu_sparse_mla import kernel_groups
    from titan_mla import _choose_num_kv_splits_mi355x, triton_mla_sparse_attention
    rng = np.random.default_rng(8101)
    g = W.gen(cuda, 8102)
    cu = torch.cuda.get_device_properties(cuda).multi_processor_count
    for case in range(CASES):
        n = int(rng.choice(list(caches)))
        kv, rows, scale = caches[n]
        T = int(rng.choice([1, 2, 3, 4, 5, 6, 7, 8, 9, 12, 16, 24, 33]))
        H = int(rng.choice([16, 16, 16, 1, 5, 15, 17, 32, 40]))
        topk = 32 * int(rng.integers(1, 90))
        pick = rng.choice([0, 0, 1, 2, 3, 5, 8, 16, 17, 23, 34, 68, int(rng.integers(1, 100))])
        splits = int(pick) or None
        idx = torch.from_numpy(rng.integers(-3, n + 5, size=(T, 1, topk)).astype(np.int32)).to(cuda)
        if rng.random() < 0.2:
            idx[:, :, int(rng.integers(0, topk)):] = -1
        q = (torch.randn(T, H, 512, generator=g, device=cuda) * float(rng.choice([0.1, 1.0, 4.0]))).to(torch.bfloat16)
        tag = ("random mla", case, n, T, H, topk, splits)
        log_case(*tag)
        out = triton_mla_sparse_attention(q, kv, idx, W.SM_SCALE, num_kv_splits=splits)
        torch.cuda.synchronize()
        S = splits or _choose_num_kv_splits_mi355x(T, -(-H // 16), topk, cu)
        want = oracle.sparse_mla(u16(q), rows, idx.cpu().numpy(), W.SM_SCALE, n_splits=S,
                                 groups=kernel_groups(topk, S), block_n=32, lazy=0.0,
                                 nthreads=oracle.default_threads())
        check_bar(out.float().cpu().numpy() / scale, bf16_to_f32(want) / scale, tag)


def test_topk_random(cuda, oracle):
    from sparse_indexer import indexer_topk
    rng = np.random.default_rng(8201)
    g = W.gen(cuda, 8202)
    for case in range(CASES):
        n = int(rng.choice([rng.integers(1, 3000), rng.integers(3000, 70000), rng.integers(60000, 140000)]))
        k = min(n, int(rng.choice([512, 512, int(rng.integers(1, min(n, 4096) + 1))])))
        R = int(rng.choice([1, 1, 2, 3, 8, 9, 16, 33]))
        x = torch.randn(R, n, generator=g, device=cuda)
        if rng.random() < 0.4:
            x = torch.round(x * float(rng.choice([1, 4, 64])))      # ties
        if rng.random() < 0.1:
            x[:, ::7] = float("nan")
        if rng.random() < 0.1:
            x[:, ::5] = float("-inf")
        lens = torch.from_numpy(rng.integers(-2, n + 3, size=R).astype(np.int32)).to(cuda)
        log_case("random top-k", case, R, n, k)
        got = indexer_topk(x, lens, k)
        torch.cuda.synchronize()
        want = oracle.indexer_topk(x.cpu().numpy(), lens.cpu().numpy(), k)
        assert np.array_equal(got.cpu().numpy(), want), (case, R, n, k)


def test_moe_align_random(cuda, oracle):
    from titan_moe_align import titan_moe_align_small
    rng = np.random.default_rng(8301)
    for case in range(CASES):
        B = int(rng.choice([1, 2, 4, 8, 3, 5, 6, 7]))
        dtype = torch.int32 if rng.random() < 0.5 else torch.int64
        ids = rng.integers(0, 288, size=(B, 8)) if rng.random() < 0.5 else rng.integers(-3, 300, size=(B, 8))
        if rng.random() < 0.3:
            ids[:] = int(rng.integers(0, 288))
        log_case("random moe align", case, B, dtype)
        got = [a.cpu().numpy() for a in titan_moe_align_small(torch.from_numpy(ids).to(dtype).to(cuda))]
        for a, b in zip(got, oracle.moe_align(ids)):
            assert a.shape == b.shape and np.array_equal(a, b), (case, B)


def test_store_int8_random(cuda, oracle):
    from titan_kv import store_int8
    rng = np.random.default_rng(8401)
    g = W.gen(cuda, 8402)
    for case in range(CASES):
        n = int(rng.integers(1, 6000))
        wide = int(rng.choice([512, 520, 1024]))
        x = (torch.randn(n, wide, generator=g, device=cuda) * float(rng.choice([1e-3, 1.0, 100.0])))
        x = x.to(torch.bfloat16)[:, :512]
        if rng.random() < 0.1:
            x[0] = 0
        nb = int(rng.integers(-(-n // 256), -(-n // 256) + 3))
        cache = torch.from_numpy(rng.integers(-128, 128, size=(nb, 256, 528)).astype(np.int8)).to(cuda)
        slots = torch.from_numpy(rng.permutation(nb * 256)[:n]).to(cuda)
        if rng.random() < 0.3:
            slots[::3] = -1
        if rng.random() < 0.5:
            slots = slots.to(torch.int32)
        want = cache.cpu().numpy().view(np.uint8).copy()
        log_case("random writer", case, n, wide, nb)
        store_int8(x, cache, slots)
        torch.cuda.synchronize()
        oracle.store_int8(u16(x), want, slots.cpu().numpy().astype(np.int64), nthreads=oracle.default_threads())
        assert np.array_equal(cache.cpu().numpy().view(np.uint8), want), (case, n, wide)
