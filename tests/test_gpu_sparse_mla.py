"""GPU parity of triton_mla_sparse_attention (HIP) against the CPU oracle.

Bar (BF16 attention output), the target one: mean-abs <= 2e-3 and per
element |err| <= 2e-2, where rare elements with |ref| >= 2 may differ by up to
two bf16 ulps of the reference value instead (rounding flips; see compare),
against
  * the reference's own reduction: one online-softmax stream per split at
    the reference's autotuned tile widths (BLOCK_N 32 and 64,
    kernels/titan_mla.py:39-43) and at the split counts the reference picks
    for these shapes on its 70-SM part (_choose_num_kv_splits: 32 at B=1,
    8 at B=8, 1 at T=2048), on the benchmark configurations exactly (the
    16384-row fixture, the 262144-row N(0,1) cache at B=1, the Student-t
    cache at B=8, all 2048 tokens of the prefill-shaped call); and
  * the oracle run with the kernel's own split count and reduction structure
    (32-key tiles dealt alternately to two key-group streams, merged at the
    end) for the edge cases (odd head counts, empty and oversubscribed
    splits, random shapes).
Plus the reference's own statistical checks against fp32 attention over the
original BF16 latents (tests/verify_mla.py:71-94) and float64 textbook
attention."""
import numpy as np
import pytest
import torch

import workloads as W
from conftest import log_case
from mla_bar import check_bar

pytestmark = pytest.mark.gpu

GROUPS = 2      # key groups of the HIP kernel: independent online-softmax streams per split
BLOCK = 32      # keys per tile
LAZY = 0.0      # the running max moves on every increase, as in the reference


def u16(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def kernel_groups(topk, splits):
    """Online-softmax streams per split in the HIP kernel for this split
    length: one past a chunk of 256 keys (the pair kernel) and for splits of
    one 32-key tile (one key group), three key groups for splits of exactly
    three tiles, two otherwise."""
    split_len = -(-topk // splits)
    return 1 if split_len > 256 or split_len <= 32 else 3 if 64 < split_len <= 96 else GROUPS


def rows_np(cache):
    return cache.contiguous().view(torch.uint8).cpu().numpy().reshape(-1, 528)


def f32(u):
    from oracle import bf16_to_f32
    return bf16_to_f32(u)


def compare(out, want_u16, tag, config=None):
    """The attention bar of mla_bar.check_bar, for a HIP output tensor against
    the oracle's bf16 bits (config: the benchmark configuration it covers)."""
    return check_bar(out.float().cpu().numpy(), f32(want_u16), tag, config=config)


def textbook_check(out, ref64, tag):
    """Against float64 softmax attention over the dequantised rows: relative
    bars (the bf16 output and bf16(p * scale) operand carry 2^-9 relative
    rounding, so heavy-tailed rows make absolute errors scale with |out|)."""
    got = out.float().cpu().numpy().astype(np.float64)
    nmse = ((got - ref64) ** 2).sum() / (ref64 ** 2).sum()
    cos = (got * ref64).sum() / np.sqrt((got ** 2).sum() * (ref64 ** 2).sum())
    print(f"[f64] {tag}: nmse {nmse:.3g} cos {cos:.8f}", flush=True)
    assert nmse < 1e-4 and cos > 0.99995, (tag, nmse, cos)


@pytest.fixture(scope="module")
def small_cache(cuda, oracle):
    from titan_kv import store_int8
    w = W.writer_small(cuda, seed=W.SEED_FIXTURE)
    store_int8(w["x"], w["cache"], w["slots"])
    torch.cuda.synchronize()
    return w, rows_np(w["cache"])


@pytest.mark.parametrize("splits", [1, 2, 4, 8, 16, 17, 32, 68, 100])
def test_small_b1_splits(cuda, oracle, small_cache, splits):
    from titan_mla import triton_mla_sparse_attention
    w, rows = small_cache
    log_case("mla small B1 splits", splits)
    n = w["n_rows"]
    out = triton_mla_sparse_attention(w["q"], w["cache"].view(n, 1, 528), w["idx"], W.SM_SCALE,
                                      num_kv_splits=splits)
    torch.cuda.synchronize()
    want = oracle.sparse_mla(u16(w["q"]), rows, w["idx"].cpu().numpy(), W.SM_SCALE, n_splits=splits,
                             groups=kernel_groups(w["idx"].shape[-1], splits), block_n=BLOCK, lazy=LAZY)
    mx, mean = compare(out, want, f"splits={splits}", config="rows16384_b1")
    assert mean < 1e-4        # ~bf16 ulp-level agreement


def test_small_auto_splits_and_graph(cuda, oracle, small_cache):
    from titan_mla import triton_mla_sparse_attention, _choose_num_kv_splits_mi355x
    w, rows = small_cache
    log_case("mla small auto + graph")
    n = w["n_rows"]
    kv = w["cache"].view(n, 1, 528)
    out = triton_mla_sparse_attention(w["q"], kv, w["idx"], W.SM_SCALE)
    s = _choose_num_kv_splits_mi355x(1, 1, 2176, torch.cuda.get_device_properties(0).multi_processor_count)
    want = oracle.sparse_mla(u16(w["q"]), rows, w["idx"].cpu().numpy(), W.SM_SCALE, n_splits=s,
                             groups=kernel_groups(w["idx"].shape[-1], s), block_n=BLOCK, lazy=LAZY)
    compare(out, want, "auto")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gout = triton_mla_sparse_attention(w["q"], kv, w["idx"], W.SM_SCALE)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(gout, out)


def test_partials_then_merge_equals_one_call(cuda, small_cache):
    """The exposed two stages reproduce glm53_sparse_mla bit for bit."""
    from titan_mla import triton_mla_sparse_attention, sparse_mla_partials, sparse_mla_merge
    w, _ = small_cache
    n = w["n_rows"]
    kv = w["cache"].view(n, 1, 528)
    g = W.gen(cuda, 5)
    q = torch.randn(3, 20, 512, generator=g, device=cuda).to(torch.bfloat16)
    idx = torch.randint(-9, n, (3, 1, 2176), generator=g, device=cuda, dtype=torch.int32)
    for s in (1, 4, 17, 68):
        log_case("mla partials+merge", s)
        full = triton_mla_sparse_attention(q, kv, idx, W.SM_SCALE, num_kv_splits=s)
        part = sparse_mla_partials(q, kv, idx, W.SM_SCALE, s)
        two = sparse_mla_merge(part, 3, 20, s)
        torch.cuda.synchronize()
        assert torch.equal(full, two), s


def test_reference_verify_protocol(cuda):
    """tests/verify_mla.py:71-94 at 65536 rows: B in {1, 6, 8}, q x 0.15,
    partial -1 padding, a positive out-of-range index; fp32 attention over the
    ORIGINAL bf16 latents; NMSE < 1e-3, cosine > 0.999; all -1 -> exactly 0."""
    from titan_kv import store_int8
    from titan_mla import triton_mla_sparse_attention
    n = 65536
    g = W.gen(cuda, W.SEED_FIXTURE)
    orig = torch.randn(n, 512, device=cuda, dtype=torch.bfloat16, generator=g)
    orig[:, :128] *= 0.05
    orig[:, 256:384] *= 8
    orig[0] = 0
    cache = torch.zeros(n // 256, 256, 528, device=cuda, dtype=torch.int8)
    store_int8(orig, cache, torch.arange(n, device=cuda, dtype=torch.int64))
    kv = cache.view(n, 1, 528)
    for batch in (1, 6, 8):
        q = torch.randn(batch, 16, 512, generator=g, device=cuda, dtype=torch.bfloat16) * 0.15
        idx = torch.randint(n, (batch, 1, 2176), generator=g, device=cuda, dtype=torch.int32)
        idx[:, :, 2048:] = -1
        if batch > 1:
            idx[1, :, 2000:] = -1
        idx[0, 0, 0] = n + 5
        valid = (idx[:, 0] >= 0) & (idx[:, 0] < n)
        chosen = orig[idx[:, 0].clamp(0, n - 1).long()].float()
        chosen.masked_fill_(~valid[:, :, None], 0)
        logits = torch.bmm(q.float(), chosen.transpose(1, 2).contiguous()) * (512 ** -0.5)
        logits.masked_fill_(~valid[:, None, :], -float("inf"))
        ref = torch.bmm(logits.softmax(-1), chosen)
        for splits in (1, 4, 8, 16, None):
            log_case("mla verify protocol", batch, splits)
            out = triton_mla_sparse_attention(q, kv, idx, 512 ** -0.5, num_kv_splits=splits)
            nmse = ((out.float() - ref).square().sum() / ref.square().sum()).item()
            cos = torch.nn.functional.cosine_similarity(out.float().flatten(), ref.flatten(), dim=0).item()
            assert bool(torch.isfinite(out).all()) and nmse < 1e-3 and cos > 0.999, (batch, splits, nmse, cos)
            blank = triton_mla_sparse_attention(q, kv, torch.full_like(idx, -1), 512 ** -0.5,
                                                num_kv_splits=splits)
            assert torch.equal(blank, torch.zeros_like(blank)), (batch, splits)


def test_head_counts_and_edges(cuda, oracle, small_cache):
    from titan_mla import triton_mla_sparse_attention
    w, rows = small_cache
    n = w["n_rows"]
    kv = w["cache"].view(n, 1, 528)
    g = W.gen(cuda, 3)
    for heads, topk, splits in ((8, 256, 1), (20, 256, 3), (32, 512, 4), (16, 32, 1), (16, 64, 5)):
        log_case("mla heads/topk/splits", heads, topk, splits)
        q = torch.randn(3, heads, 512, generator=g, device=cuda).to(torch.bfloat16)
        idx = torch.randint(-50, n + 50, (3, 1, topk), generator=g, device=cuda, dtype=torch.int32)
        out = triton_mla_sparse_attention(q, kv, idx, W.SM_SCALE, num_kv_splits=splits)
        torch.cuda.synchronize()
        want = oracle.sparse_mla(u16(q), rows, idx.cpu().numpy(), W.SM_SCALE, n_splits=splits,
                                 groups=kernel_groups(idx.shape[-1], splits), block_n=BLOCK, lazy=LAZY)
        compare(out, want, (heads, topk, splits))
    # int64 indices, including values that alias valid rows modulo 2^32
    q = torch.randn(2, 16, 512, generator=g, device=cuda).to(torch.bfloat16)
    idx64 = torch.randint(0, n, (2, 1, 256), generator=g, device=cuda, dtype=torch.int64)
    idx64[0, 0, :40] += 1 << 32
    out = triton_mla_sparse_attention(q, kv, idx64, W.SM_SCALE, num_kv_splits=2)
    clean = torch.where((idx64 >= 0) & (idx64 < n), idx64, -1).to(torch.int32)
    want = oracle.sparse_mla(u16(q), rows, clean.cpu().numpy(), W.SM_SCALE, n_splits=2,
                             groups=kernel_groups(clean.shape[-1], 2), block_n=BLOCK, lazy=LAZY)
    compare(out, want, "int64")
    # no tokens
    empty = triton_mla_sparse_attention(q[:0], kv, idx64[:0].to(torch.int32), W.SM_SCALE)
    assert empty.shape == (0, 16, 512)


def test_random_shapes(cuda, oracle, small_cache):
    """Seeded random token counts, head counts, top-k, split counts and index
    sets (pads, out-of-range values both ways, repeated rows), each against
    the oracle with the kernel's split count."""
    from titan_mla import triton_mla_sparse_attention, _choose_num_kv_splits_mi355x
    w, rows = small_cache
    n = w["n_rows"]
    kv = w["cache"].view(n, 1, 528)
    rng = np.random.default_rng(4242)
    g = W.gen(cuda, 4242)
    for case in range(40):
        T = int(rng.integers(1, 7))
        heads = int(rng.choice([1, 4, 8, 16, 20, 32]))
        topk = 32 * int(rng.integers(1, 81))
        splits = int(rng.choice([0, 1, 2, 3, 5, 8, 17, 40]))
        q = (torch.randn(T, heads, 512, generator=g, device=cuda) * float(rng.uniform(0.05, 1.5))).to(torch.bfloat16)
        idx = torch.from_numpy(rng.integers(-40, n + 40, size=(T, 1, topk)).astype(np.int32)).to(cuda)
        if case % 4 == 1:
            idx[:, :, topk // 2:] = -1                                  # trailing pads
        if case % 4 == 2:
            idx[:, :, : topk // 3] = idx[:, :, :1]                      # one row repeated
        eff = splits or _choose_num_kv_splits_mi355x(T, -(-heads // 16), topk, 256)
        log_case("mla random", case, T, heads, topk, splits, eff)
        out = triton_mla_sparse_attention(q, kv, idx, W.SM_SCALE, num_kv_splits=splits or None, sm_count=256)
        torch.cuda.synchronize()
        want = oracle.sparse_mla(u16(q), rows, idx.cpu().numpy(), W.SM_SCALE, n_splits=eff,
                                 groups=kernel_groups(idx.shape[-1], eff),
                                 block_n=BLOCK, lazy=LAZY)
        compare(out, want, ("random", case, T, heads, topk, eff))


def test_xcd_grouped_units(cuda, oracle, small_cache):
    """Unit counts (tokens x head groups) that are a multiple of 8 take the
    XCD-grouped workgroup numbering in the split and merge kernels: 8 tokens
    x 1 group, 4 tokens x 2 groups (32 heads), 8 tokens x 4 groups (64
    heads) and 16 tokens x 1 group, each with several splits, against the
    oracle; 20 heads (padded group) at 8 tokens too."""
    from titan_mla import triton_mla_sparse_attention
    w, rows = small_cache
    n = w["n_rows"]
    kv = w["cache"].view(n, 1, 528)
    rng = np.random.default_rng(808)
    g = W.gen(cuda, 808)
    for T, heads, topk, splits in ((8, 16, 2176, 17), (4, 32, 1024, 8), (8, 64, 512, 4), (16, 16, 640, 5),
                                   (8, 20, 896, 7)):
        q = torch.randn(T, heads, 512, generator=g, device=cuda).to(torch.bfloat16)
        idx = torch.from_numpy(rng.integers(-8, n + 8, size=(T, 1, topk)).astype(np.int32)).to(cuda)
        log_case("mla xcd-grouped", T, heads, topk, splits)
        out = triton_mla_sparse_attention(q, kv, idx, W.SM_SCALE, num_kv_splits=splits)
        torch.cuda.synchronize()
        want = oracle.sparse_mla(u16(q), rows, idx.cpu().numpy(), W.SM_SCALE, n_splits=splits,
                                 groups=kernel_groups(idx.shape[-1], splits), block_n=BLOCK, lazy=LAZY)
        compare(out, want, ("xcd-grouped", T, heads, topk, splits))


def test_padded_token_numbering(cuda, oracle, small_cache):
    """Batches of 3, 5, 6 and 7 tokens (one head group) are numbered as 4 or 8
    tokens by the split and merge kernels when each token's splits fit its
    XCDs (the extra tokens' workgroups return at once): the auto split count
    (34 at 3 tokens, 23 at 5-7), forced counts that still pad (17; 34 at 3)
    and ones that do not (34 at 5-7: more than one XCD's CUs; one-tile
    splits), each against the oracle, and the partials + merge path equal to
    the one call byte for byte."""
    from titan_mla import (triton_mla_sparse_attention, sparse_mla_partials, sparse_mla_merge,
                           _choose_num_kv_splits_mi355x)
    w, rows = small_cache
    n = w["n_rows"]
    kv = w["cache"].view(n, 1, 528)
    rng = np.random.default_rng(909)
    g = W.gen(cuda, 909)
    cu = torch.cuda.get_device_properties(cuda).multi_processor_count
    for T in (3, 5, 6, 7):
        topk = 2176
        q = torch.randn(T, 16, 512, generator=g, device=cuda).to(torch.bfloat16)
        idx = torch.from_numpy(rng.integers(-8, n + 8, size=(T, 1, topk)).astype(np.int32)).to(cuda)
        auto = _choose_num_kv_splits_mi355x(T, 1, topk, cu)
        assert auto == (34 if T == 3 else 23)
        for splits in (auto, 17, 34, 68):
            log_case("mla padded numbering", T, topk, splits)
            out = triton_mla_sparse_attention(q, kv, idx, W.SM_SCALE, num_kv_splits=splits)
            parts = sparse_mla_merge(sparse_mla_partials(q, kv, idx, W.SM_SCALE, splits), T, 16, splits)
            torch.cuda.synchronize()
            assert torch.equal(parts, out), ("partials + merge", T, splits)
            want = oracle.sparse_mla(u16(q), rows, idx.cpu().numpy(), W.SM_SCALE, n_splits=splits,
                                     groups=kernel_groups(topk, splits), block_n=BLOCK, lazy=LAZY)
            compare(out, want, ("padded numbering", T, splits))


@pytest.fixture(scope="module")
def full_cache(cuda):
    from titan_kv import store_int8
    g, x, cache, slots = W.decode_cache(cuda, seed=W.SEED_BENCH, dist="t3")
    store_int8(x, cache, slots)
    torch.cuda.synchronize()
    del x
    return g, cache


@pytest.mark.slow
def test_full_context_b1_b8(cuda, oracle, full_cache):
    """262144-row cache: B=1 with 2048 uniform + 128 pads, B=8 locality-biased
    with 0..256 pads per row (Student-t latents stress per-row scales)."""
    from titan_mla import triton_mla_sparse_attention, _choose_num_kv_splits_mi355x
    g, cache = full_cache
    n = cache.shape[0] * 256
    kv = cache.view(n, 1, 528)
    rows = rows_np(cache)
    cu = torch.cuda.get_device_properties(0).multi_processor_count
    for name, (q, idx) in (("b1", W.decode_b1_inputs(cuda, g)), ("b8", W.decode_b8_inputs(cuda, g))):
        for splits in (None, 1, 8):
            log_case("mla full context", name, splits)
            out = triton_mla_sparse_attention(q, kv, idx, W.SM_SCALE, num_kv_splits=splits)
            torch.cuda.synchronize()
            s = splits or _choose_num_kv_splits_mi355x(q.shape[0], 1, 2176, cu)
            want = oracle.sparse_mla(u16(q), rows, idx.cpu().numpy(), W.SM_SCALE, n_splits=s,
                                     nthreads=oracle.default_threads(), groups=kernel_groups(idx.shape[-1], s),
                                     block_n=BLOCK, lazy=LAZY)
            compare(out, want, (name, splits), config="rows262144_t3_b8" if name == "b8" else None)
            ref64 = oracle.sparse_mla_f64(u16(q), rows, idx.cpu().numpy(), W.SM_SCALE,
                                          nthreads=oracle.default_threads())
            textbook_check(out, ref64, (name, splits))


@pytest.mark.slow
def test_prefill_shaped_sampled(cuda, oracle, full_cache):
    """T = 2048 query tokens, causal locality-biased indices; the oracle checks
    a sample of 48 tokens (first, last and random)."""
    from titan_mla import triton_mla_sparse_attention
    g, cache = full_cache
    n = cache.shape[0] * 256
    kv = cache.view(n, 1, 528)
    rows = rows_np(cache)
    q, idx, _, _ = W.prefill_inputs(cuda, g)
    log_case("mla prefill-shaped T=2048")
    out = triton_mla_sparse_attention(q, kv, idx, W.SM_SCALE)
    torch.cuda.synchronize()
    pick = np.unique(np.concatenate([[0, 1, 2047], np.random.default_rng(0).integers(0, 2048, 45)]))
    qs = u16(q)[pick]
    ids = idx.cpu().numpy()[pick]
    want = oracle.sparse_mla(qs, rows, ids, W.SM_SCALE, n_splits=1, nthreads=oracle.default_threads(),
                             groups=kernel_groups(idx.shape[-1], 1), block_n=BLOCK, lazy=LAZY)
    got = out[torch.as_tensor(pick, device=cuda)]
    compare(got, want, "prefill sample", config="prefill_t2048")


# ---------------------------------------------------------------- the reference's own reduction

REF_SM_COUNT = 70        # the reference's part (integration/titan_backend.py:28)


def ref_splits(tokens):
    """The split count the reference's heuristic picks on its own part
    (kernels/titan_mla.py:432-449): 32 at B=1, 8 at B=8, 1 at T=2048."""
    from titan_mla import _choose_num_kv_splits
    return _choose_num_kv_splits(tokens, 1, W.TOPK, REF_SM_COUNT)


def check_reference_reduction(oracle, outs, q, rows, idx, tag, config=None):
    """Every GPU output in `outs` against the reference's single-stream
    reduction at both autotuned tile widths and the reference's split count."""
    s = ref_splits(q.shape[0])
    qn, ixn = u16(q), idx.cpu().numpy()
    for block_n in (32, 64):
        want = oracle.sparse_mla(qn, rows, ixn, W.SM_SCALE, n_splits=s, groups=1, block_n=block_n,
                                 nthreads=oracle.default_threads())
        for name, out in outs.items():
            compare(out, want, (tag, name, f"reference splits={s} BLOCK_N={block_n}"), config=config)


def test_reference_reduction_small(cuda, oracle, small_cache):
    """The 16384-row fixture at B=1 (2048 uniform + 128 pads)."""
    from titan_mla import triton_mla_sparse_attention
    w, rows = small_cache
    n = w["n_rows"]
    kv = w["cache"].view(n, 1, 528)
    log_case("mla small B1 vs the reference reduction")
    outs = {"auto": triton_mla_sparse_attention(w["q"], kv, w["idx"], W.SM_SCALE),
            "reference splits": triton_mla_sparse_attention(w["q"], kv, w["idx"], W.SM_SCALE,
                                                            num_kv_splits=ref_splits(1))}
    torch.cuda.synchronize()
    check_reference_reduction(oracle, outs, w["q"], rows, w["idx"], "small B1", config="rows16384_b1")


@pytest.fixture(scope="module")
def normal_cache(cuda):
    """262144 rows of N(0,1) latents: the full-context B=1 configuration."""
    from titan_kv import store_int8
    g, x, cache, slots = W.decode_cache(cuda, seed=W.SEED_BENCH + 1, dist="normal")
    store_int8(x, cache, slots)
    torch.cuda.synchronize()
    del x
    return cache, rows_np(cache)


@pytest.mark.slow
def test_reference_reduction_full_b1(cuda, oracle, normal_cache):
    """B=1 over the N(0,1) 262144-row cache: 2048 indices uniform over the
    context, then 128 pads."""
    from titan_mla import triton_mla_sparse_attention
    cache, rows = normal_cache
    kv = cache.view(-1, 1, 528)
    q, idx = W.decode_b1_inputs(cuda, W.gen(cuda, W.SEED_BENCH + 11))
    assert int((idx >= 0).sum()) == 2048
    log_case("mla full B1 N(0,1) vs the reference reduction")
    outs = {"auto": triton_mla_sparse_attention(q, kv, idx, W.SM_SCALE),
            "reference splits": triton_mla_sparse_attention(q, kv, idx, W.SM_SCALE, num_kv_splits=ref_splits(1))}
    torch.cuda.synchronize()
    check_reference_reduction(oracle, outs, q, rows, idx, "full B1", config="rows262144_normal_b1")


@pytest.mark.slow
def test_reference_reduction_full_b8(cuda, oracle, full_cache):
    """B=8 over the Student-t 262144-row cache, locality-biased indices with
    0..256 trailing pads per row."""
    from titan_mla import triton_mla_sparse_attention
    _, cache = full_cache
    kv = cache.view(-1, 1, 528)
    rows = rows_np(cache)
    q, idx = W.decode_b8_inputs(cuda, W.gen(cuda, W.SEED_BENCH + 18))
    log_case("mla full B8 Student-t vs the reference reduction")
    outs = {"auto": triton_mla_sparse_attention(q, kv, idx, W.SM_SCALE),
            "reference splits": triton_mla_sparse_attention(q, kv, idx, W.SM_SCALE, num_kv_splits=ref_splits(8))}
    torch.cuda.synchronize()
    check_reference_reduction(oracle, outs, q, rows, idx, "full B8", config="rows262144_t3_b8")


@pytest.mark.slow
def test_reference_reduction_prefill_all_tokens(cuda, oracle, full_cache):
    """The prefill-shaped call, every one of its 2048 query tokens: causal
    locality-biased indices over the Student-t cache, one split (the
    reference's choice and the library's)."""
    from titan_mla import triton_mla_sparse_attention
    _, cache = full_cache
    kv = cache.view(-1, 1, 528)
    rows = rows_np(cache)
    q, idx, _, _ = W.prefill_inputs(cuda, W.gen(cuda, W.SEED_BENCH + 2048))
    assert ref_splits(2048) == 1
    log_case("mla prefill-shaped T=2048, all tokens, vs the reference reduction")
    outs = {"auto": triton_mla_sparse_attention(q, kv, idx, W.SM_SCALE)}
    torch.cuda.synchronize()
    check_reference_reduction(oracle, outs, q, rows, idx, "prefill T=2048", config="prefill_t2048")


def test_merge_beyond_register_splits(cuda, oracle, small_cache):
    """More than 128 splits take the merge kernel's loop path (the register
    path holds 128): 200 and 256 splits of a 16384-index top-k (the auto
    policy's answer at B=1), against the oracle with the same splits, and
    partials + merge equal to one call bit for bit."""
    from titan_mla import (triton_mla_sparse_attention, sparse_mla_partials, sparse_mla_merge,
                           _choose_num_kv_splits_mi355x)
    w, rows = small_cache
    n = w["n_rows"]
    kv = w["cache"].view(n, 1, 528)
    g = W.gen(cuda, 16384)
    q = torch.randn(2, 16, 512, generator=g, device=cuda).to(torch.bfloat16)
    idx = torch.randint(-64, n, (2, 1, 16384), generator=g, device=cuda, dtype=torch.int32)
    assert _choose_num_kv_splits_mi355x(1, 1, 16384, 256) == 256
    for s in (200, 256):
        log_case("mla merge loop path", s)
        out = triton_mla_sparse_attention(q, kv, idx, W.SM_SCALE, num_kv_splits=s)
        two = sparse_mla_merge(sparse_mla_partials(q, kv, idx, W.SM_SCALE, s), 2, 16, s)
        torch.cuda.synchronize()
        assert torch.equal(out, two), s
        want = oracle.sparse_mla(u16(q), rows, idx.cpu().numpy(), W.SM_SCALE, n_splits=s,
                                 groups=kernel_groups(idx.shape[-1], s), block_n=BLOCK, lazy=LAZY,
                                 nthreads=oracle.default_threads())
        compare(out, want, ("merge loop path", s))


def test_gather_floor_diagnostic(cuda, small_cache):
    """The memory-chain probe runs on the decode grids of every split-kernel
    shape, fills the whole partials buffer the merge reads (junk, finite),
    and refuses splits longer than one chunk of gathers."""
    from titan_mla import sparse_mla_gather_floor, sparse_mla_merge
    w, _ = small_cache
    n = w["n_rows"]
    kv = w["cache"].view(n, 1, 528)
    g = W.gen(cuda, 21)
    q = torch.randn(8, 16, 512, generator=g, device=cuda).to(torch.bfloat16)
    idx = torch.randint(-8, n, (8, 1, 2176), generator=g, device=cuda, dtype=torch.int32)
    for s in (17, 34, 23, 68):   # two key groups, three (95-key splits), one (32-key splits)
        log_case("gather floor", s)
        buf = sparse_mla_gather_floor(q, kv, idx, s)
        out = sparse_mla_merge(buf, 8, 16, s)
        torch.cuda.synchronize()
        assert bool(torch.isfinite(buf.view(torch.float32)).all()) and out.shape == (8, 16, 512)
    with pytest.raises(RuntimeError):
        sparse_mla_gather_floor(q, kv, idx, 1)
    with pytest.raises(RuntimeError):   # masked keys read row 0: an empty cache is refused
        sparse_mla_gather_floor(q, kv[:0], idx, 68)


def test_split_length_boundaries(cuda, oracle, small_cache):
    """Split lengths at every boundary between the kernel variants, 2176
    indices with pads and out-of-range values: 32 keys (one key group), 33
    and 64 (two groups, one round), 66 and 95 (three groups), 99 and 242 (two
    groups, two to eight tiles), 272 (the pair kernel) -- each against the
    oracle with the same stream structure."""
    from titan_mla import triton_mla_sparse_attention
    w, rows = small_cache
    n = w["n_rows"]
    kv = w["cache"].view(n, 1, 528)
    g = W.gen(cuda, 321)
    T, H, topk = 2, 16, 2176
    q = torch.randn(T, H, 512, generator=g, device=cuda).to(torch.bfloat16)
    idx = torch.randint(-40, n + 40, (T, 1, topk), generator=g, device=cuda, dtype=torch.int32)
    idx[1, :, 1900:] = -1
    for splits, split_len in ((68, 32), (66, 33), (34, 64), (33, 66), (23, 95), (22, 99), (9, 242), (8, 272)):
        assert -(-topk // splits) == split_len
        log_case("mla split-length boundary", splits, split_len)
        out = triton_mla_sparse_attention(q, kv, idx, W.SM_SCALE, num_kv_splits=splits)
        torch.cuda.synchronize()
        want = oracle.sparse_mla(u16(q), rows, idx.cpu().numpy(), W.SM_SCALE, n_splits=splits,
                                 groups=kernel_groups(topk, splits), block_n=BLOCK, lazy=LAZY)
        mx, mean = compare(out, want, ("split length", splits, split_len))
        assert mean < 1e-4
    # single splits written as bf16 directly: one tile (one key group), three
    # tiles (three key groups), and 20 heads (a padded head group)
    for topk, heads in ((32, 16), (96, 16), (32, 20), (96, 20)):
        q = torch.randn(3, heads, 512, generator=g, device=cuda).to(torch.bfloat16)
        idx = torch.randint(-8, n + 8, (3, 1, topk), generator=g, device=cuda, dtype=torch.int32)
        log_case("mla single split", topk, heads)
        out = triton_mla_sparse_attention(q, kv, idx, W.SM_SCALE, num_kv_splits=1)
        torch.cuda.synchronize()
        want = oracle.sparse_mla(u16(q), rows, idx.cpu().numpy(), W.SM_SCALE, n_splits=1,
                                 groups=kernel_groups(topk, 1), block_n=BLOCK, lazy=LAZY)
        mx, mean = compare(out, want, ("single split", topk, heads))
        assert mean < 1e-4


def test_three_key_group_splits(cuda, oracle, small_cache):
    """Splits of exactly three 32-key tiles (65 to 96 indices) run on the
    12-wave variant (three key-group streams, one round): against the oracle
    with the same three streams and, within the bar, the reference's single
    stream; a single split writing bf16 directly (96 indices), a padded head
    group (20 heads), ragged last splits (224 in 3, 352 in 4, 2176 in 23 and
    24 -- B=8's split policy), pads and indices outside the cache both ways;
    all -1 gives exactly 0; the paged form of the same call is bit-identical
    to the flat one."""
    from titan_mla import triton_mla_sparse_attention, triton_mla_sparse_attention_paged
    w, rows = small_cache
    n = w["n_rows"]
    kv = w["cache"].view(n, 1, 528)
    g = W.gen(cuda, 123)
    for T, H, topk, splits in ((3, 16, 96, 1), (2, 20, 224, 3), (5, 16, 352, 4), (8, 16, 2176, 23),
                               (4, 16, 2176, 24)):
        assert kernel_groups(topk, splits) == 3
        q = torch.randn(T, H, 512, generator=g, device=cuda).to(torch.bfloat16)
        idx = torch.randint(-40, n + 40, (T, 1, topk), generator=g, device=cuda, dtype=torch.int32)
        idx[0, :, topk // 2:] = -1
        log_case("mla three key groups", T, H, topk, splits)
        out = triton_mla_sparse_attention(q, kv, idx, W.SM_SCALE, num_kv_splits=splits)
        torch.cuda.synchronize()
        want = oracle.sparse_mla(u16(q), rows, idx.cpu().numpy(), W.SM_SCALE, n_splits=splits, groups=3,
                                 block_n=BLOCK, lazy=LAZY)
        mx, mean = compare(out, want, ("three groups", T, H, topk, splits))
        assert mean < 1e-4        # ~bf16 ulp-level agreement with its own reduction structure
        single = oracle.sparse_mla(u16(q), rows, idx.cpu().numpy(), W.SM_SCALE, n_splits=splits, groups=1,
                                   block_n=BLOCK)
        compare(out, single, ("three groups vs single stream", T, H, topk, splits))
        blank = triton_mla_sparse_attention(q, kv, torch.full_like(idx, -1), W.SM_SCALE, num_kv_splits=splits)
        assert torch.equal(blank, torch.zeros_like(blank)), (T, H, topk, splits)
    # paged: one request whose block table maps positions to the same rows
    T, H, topk, splits, bs = 4, 16, 2176, 23, 64
    q = torch.randn(T, H, 512, generator=g, device=cuda).to(torch.bfloat16)
    idx = torch.randint(-8, n + 8, (T, 1, topk), generator=g, device=cuda, dtype=torch.int32)
    flat = triton_mla_sparse_attention(q, kv, idx, W.SM_SCALE, num_kv_splits=splits)
    pages = w["cache"].view(n // bs, bs, 528)
    table = torch.arange(n // bs, device=cuda, dtype=torch.int32)[None, :]
    req = torch.zeros(T, dtype=torch.int32, device=cuda)
    paged = triton_mla_sparse_attention_paged(q, pages, idx, req, table, W.SM_SCALE, num_kv_splits=splits)
    torch.cuda.synchronize()
    assert torch.equal(paged, flat)


def test_long_split_pair_kernel_edges(cuda, oracle, small_cache):
    """Splits longer than one chunk (256 indices) run on the pair kernel (one
    online-softmax stream per split): against the reference's single stream
    (groups=1, BLOCK_N=32) with odd tile counts (352 = 11 tiles, 288 = 9), a
    last split shorter than the others (1088 in 3 splits), split partials
    merged (2176 in 2 splits, 20 heads: a padded head group), pads and
    indices outside the cache both ways; all -1 gives exactly 0; an empty
    cache (no rows) gives exactly 0 without reading it."""
    from titan_mla import triton_mla_sparse_attention
    w, rows = small_cache
    n = w["n_rows"]
    kv = w["cache"].view(n, 1, 528)
    g = W.gen(cuda, 99)
    for T, H, topk, splits in ((5, 20, 2176, 2), (3, 16, 352, 1), (2, 16, 288, 1), (4, 32, 1088, 3),
                               (3, 16, 2176, 1), (2, 16, 320, 1)):
        q = torch.randn(T, H, 512, generator=g, device=cuda).to(torch.bfloat16)
        idx = torch.randint(-40, n + 40, (T, 1, topk), generator=g, device=cuda, dtype=torch.int32)
        idx[0, :, topk // 2:] = -1
        log_case("mla pair kernel", T, H, topk, splits)
        out = triton_mla_sparse_attention(q, kv, idx, W.SM_SCALE, num_kv_splits=splits)
        torch.cuda.synchronize()
        want = oracle.sparse_mla(u16(q), rows, idx.cpu().numpy(), W.SM_SCALE, n_splits=splits, groups=1, block_n=32)
        compare(out, want, ("pair kernel", T, H, topk, splits))
        blank = triton_mla_sparse_attention(q, kv, torch.full_like(idx, -1), W.SM_SCALE, num_kv_splits=splits)
        assert torch.equal(blank, torch.zeros_like(blank)), (T, H, topk, splits)
    q = torch.randn(2, 16, 512, generator=g, device=cuda).to(torch.bfloat16)
    idx = torch.randint(0, 100, (2, 1, 1024), generator=g, device=cuda, dtype=torch.int32)
    empty = torch.zeros(0, 1, 528, dtype=torch.int8, device=cuda)
    out = triton_mla_sparse_attention(q, empty, idx, W.SM_SCALE, num_kv_splits=1)
    torch.cuda.synchronize()
    assert torch.equal(out, torch.zeros_like(out))
