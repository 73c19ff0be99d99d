"""GPU parity of titan_moe_align_small (HIP) against the CPU oracle: bit-exact
sorted_ids, expert_ids and num_tokens_post_padded, over the reference's
routing patterns (benchmarks/moe_align.py:49-55, 113-173)."""
import random

import numpy as np
import pytest
import torch

import workloads as W
from conftest import log_case
from parity_log import record_exact

pytestmark = pytest.mark.gpu


def _check(ids, want, **kw):
    from titan_moe_align import titan_moe_align_small
    got = titan_moe_align_small(ids, **kw)
    for g_, w_ in zip(got, want):
        assert g_.dtype == torch.int32
        assert np.array_equal(g_.cpu().numpy(), w_), (ids.cpu().tolist(), kw)


def test_reference_patterns_all_dtypes_and_warps(cuda, oracle):
    rng = random.Random(37)
    cases = 0
    for batch in range(1, 9):
        log_case("moe patterns", batch)
        for name, flat in oracle.moe_patterns(batch, rng).items():
            want = oracle.moe_align(flat)
            for dtype in (torch.int32, torch.int64):
                ids = torch.tensor(flat, dtype=dtype, device=cuda).view(batch, 8)
                for warps in (1, 2, 4):
                    _check(ids, want, num_warps=warps)
                    _check(ids, want, pad_sorted_ids=True, num_warps=warps)
                    cases += 1
                _check(ids, want)
    assert cases == 8 * 7 * 2 * 3


def test_random_and_invalid_routes(cuda, oracle):
    rng = random.Random(2026)
    log_case("moe random routes")
    for batch in range(1, 9):
        for _ in range(60):
            flat = [rng.randrange(-2, 292) for _ in range(batch * 8)]
            want = oracle.moe_align(flat)
            for dtype in (torch.int32, torch.int64):
                _check(torch.tensor(flat, dtype=dtype, device=cuda).view(batch, 8), want)
    # 64-bit ids that alias valid experts in their low 32 bits are invalid
    flat = [(1 << 32) + 5, 5, -(1 << 40), 287, 288, (1 << 33), 0, 7]
    _check(torch.tensor(flat, dtype=torch.int64, device=cuda).view(1, 8), oracle.moe_align(flat))


def test_distinct_topk_and_adversarial(cuda, oracle):
    from titan_moe_align import titan_moe_align_small
    g = W.gen(cuda, W.SEED_BENCH)
    for batch in (1, 2, 4, 8):
        log_case("moe distinct/adversarial", batch)
        ids = W.moe_routes(batch, cuda, g)
        shared = torch.arange(8, device=cuda, dtype=torch.int32).repeat(batch, 1)
        for case, routes in (("distinct top-8", ids), ("shared top-8", shared)):
            want = oracle.moe_align(routes.cpu().numpy())
            got = [t.cpu().numpy() for t in titan_moe_align_small(routes)]
            record_exact("moe_align_b1_b8", f"MoE align {case} (sorted_ids, expert_ids, padded count)",
                         sum(int(np.count_nonzero(a != b)) if a.shape == b.shape else a.size
                             for a, b in zip(got, want)), sum(b.size for b in want))
            if case == "shared top-8":
                assert want[2][0] == 64
            _check(routes, want)


def test_graph_replay(cuda, oracle):
    """Captured once, replayed with new ids written into the same input."""
    from titan_moe_align import titan_moe_align_small
    log_case("moe graph replay")
    ids = torch.zeros(8, 8, dtype=torch.int32, device=cuda)
    titan_moe_align_small(ids)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = titan_moe_align_small(ids)
    rng = random.Random(5)
    for _ in range(5):
        flat = [rng.randrange(-2, 292) for _ in range(64)]
        ids.copy_(torch.tensor(flat, dtype=torch.int32).view(8, 8))
        graph.replay()
        torch.cuda.synchronize()
        for g_, w_ in zip(out, oracle.moe_align(flat)):
            assert np.array_equal(g_.cpu().numpy(), w_)
