"""Pins the indexer oracle (oracle.e4m3_to_f32, fp8_paged_mqa_logits,
indexer_topk) against what fixes it independently: torch's float8_e4m3fn
decoding, closed-form logits from unit queries, the relu, paging
invariances, an independent torch formulation, and brute-force selection.
CPU only."""
import numpy as np
import pytest

D = 128


def page_layout(keys_u8, scales, block_size, page_bytes=None):
    """Fused pages [num_blocks, page_bytes] from keys [n, 128] and scales [n]
    (key i -> block i // block_size, slot i % block_size)."""
    n = keys_u8.shape[0]
    nb = (n + block_size - 1) // block_size
    page_bytes = page_bytes or block_size * (D + 4)
    pages = np.zeros((nb, page_bytes), dtype=np.uint8)
    for i in range(n):
        b, o = divmod(i, block_size)
        pages[b, o * D:(o + 1) * D] = keys_u8[i]
        pages[b, block_size * D + 4 * o: block_size * D + 4 * o + 4] = np.array([scales[i]], np.float32).view(np.uint8)
    return pages


def test_e4m3_matches_torch():
    import torch
    import oracle
    codes = np.arange(256, dtype=np.uint8)
    assert np.array_equal(oracle.e4m3_to_f32(codes), torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy(),
                          equal_nan=True)
    assert oracle.e4m3_to_f32(np.array([0x38, 0x01, 0x7E, 0xFE, 0x08]))[[0, 1, 2, 3, 4]].tolist() == \
        [1.0, 2.0 ** -9, 448.0, -448.0, 2.0 ** -6]


def test_unit_query_closed_form(oracle):
    """q = 1.0 at dim d0 of head h0 only, weight 1 on h0: logit j =
    relu(s_j * k_j[d0])."""
    rng = np.random.default_rng(1)
    n, H, bs = 200, 16, 64
    keys = rng.integers(0, 256, size=(n, D), dtype=np.uint8)
    keys[(keys & 0x7F) == 0x7F] = 0
    scales = rng.uniform(0.01, 2.0, size=n).astype(np.float32)
    pages = page_layout(keys, scales, bs)
    q = np.zeros((1, H, D), dtype=np.uint8)
    h0, d0 = 5, 77
    q[0, h0, d0] = 0x38
    w = np.zeros((1, H), np.float32)
    w[0, h0] = 1.0
    bt = np.arange(pages.shape[0], dtype=np.int32)[None, :]
    got = oracle.fp8_paged_mqa_logits(q, pages, bs, w, np.array([n]), bt, n + 10)
    kv = oracle.e4m3_to_f32(keys[:, d0]).astype(np.float64)
    want = np.maximum(scales.astype(np.float64) * kv, 0.0)
    assert np.array_equal(got[0, :n], want)
    assert np.all(np.isneginf(got[0, n:]))


def test_paging_invariance_and_masks(oracle):
    rng = np.random.default_rng(2)
    n, H, bs = 300, 32, 16
    keys = rng.integers(0, 256, size=(n, D), dtype=np.uint8)
    keys[(keys & 0x7F) == 0x7F] = 0
    scales = rng.uniform(0.01, 1.0, size=n).astype(np.float32)
    q = rng.integers(0, 256, size=(2, H, D), dtype=np.uint8)
    q[(q & 0x7F) == 0x7F] = 0
    w = rng.standard_normal((2, H)).astype(np.float32)
    pages = page_layout(keys, scales, bs, page_bytes=bs * (D + 4) + 48)
    nb = pages.shape[0]
    bt = np.tile(np.arange(nb, dtype=np.int32), (2, 1))
    ctx = np.array([n, 123])
    base = oracle.fp8_paged_mqa_logits(q, pages, bs, w, ctx, bt, n)
    # the same keys in permuted pages, read through the permuted table
    perm = rng.permutation(nb)
    pages2 = np.zeros_like(pages)
    pages2[perm] = pages
    bt2 = perm[bt].astype(np.int32)
    assert np.array_equal(oracle.fp8_paged_mqa_logits(q, pages2, bs, w, ctx, bt2, n), base, equal_nan=True)
    # a table entry outside the cache masks its page; unclean rows leave the tail unwritten
    bt3 = bt.copy()
    bt3[0, 3] = nb + 5
    got = oracle.fp8_paged_mqa_logits(q, pages, bs, w, ctx, bt3, n, clean=False)
    assert np.all(np.isneginf(got[0, 3 * bs:4 * bs]))
    assert np.array_equal(np.delete(got[0], np.arange(3 * bs, 4 * bs)), np.delete(base[0], np.arange(3 * bs, 4 * bs)))
    assert np.all(np.isnan(got[1, 123:])) and np.all(np.isneginf(base[1, 123:]))


def test_relu_and_torch_formulation(oracle):
    """An independent formulation: torch decodes the fp8 bytes, einsum,
    clamp, weighted head sum."""
    import torch
    rng = np.random.default_rng(3)
    n, H, bs, T = 257, 48, 64, 3
    keys = rng.integers(0, 256, size=(n, D), dtype=np.uint8)
    keys[(keys & 0x7F) == 0x7F] = 1
    scales = rng.uniform(0.001, 0.5, size=n).astype(np.float32)
    q = rng.integers(0, 256, size=(T, H, D), dtype=np.uint8)
    q[(q & 0x7F) == 0x7F] = 2
    w = rng.standard_normal((T, H)).astype(np.float32)
    pages = page_layout(keys, scales, bs)
    bt = np.tile(np.arange(pages.shape[0], dtype=np.int32), (T, 1))
    ctx = np.array([n, 100, 1])
    got = oracle.fp8_paged_mqa_logits(q, pages, bs, w, ctx, bt, n)
    kt = torch.from_numpy(keys).view(torch.float8_e4m3fn).double()
    qt = torch.from_numpy(q).view(torch.float8_e4m3fn).double()
    dots = torch.einsum("thd,nd->tnh", qt, kt) * torch.from_numpy(scales).double()[None, :, None]
    want = (dots.clamp(min=0) * torch.from_numpy(w).double()[:, None, :]).sum(-1).numpy()
    for t in range(T):
        assert np.allclose(got[t, :ctx[t]], want[t, :ctx[t]], rtol=1e-12, atol=1e-12)
        assert np.all(np.isneginf(got[t, ctx[t]:]))
    # the relu is active: some (head, key) dot products are negative
    assert (dots < 0).any() and (dots > 0).any()


def brute_topk(row, n, k):
    import math
    items = []
    for i in range(n):
        v = float(row[i])
        key = -math.inf if math.isnan(v) else v
        items.append((0 if math.isnan(v) else 1, key, -i))
    best = sorted(range(n), key=lambda i: items[i], reverse=True)[:k]
    return sorted(best)


def test_topk_brute_force(oracle):
    rng = np.random.default_rng(4)
    rows = []
    lens = []
    for n, kind in [(1000, "normal"), (600, "ties"), (40, "short"), (512, "exact"), (900, "specials")]:
        if kind == "ties":
            r = rng.integers(0, 5, size=1200).astype(np.float32)
        else:
            r = rng.standard_normal(1200).astype(np.float32)
        if kind == "specials":
            r[rng.integers(0, n, 50)] = np.nan
            r[rng.integers(0, n, 50)] = -np.inf
            r[rng.integers(0, n, 20)] = np.inf
            r[rng.integers(0, n, 20)] = -0.0
        rows.append(r)
        lens.append(n)
    logits = np.stack(rows)
    k = 512
    got = oracle.indexer_topk(logits, np.array(lens), k)
    for r in range(len(rows)):
        want = brute_topk(logits[r], lens[r], k)
        assert got[r, :len(want)].tolist() == want
        assert np.all(got[r, len(want):] == -1)


def test_nan_products_are_dropped(oracle):
    """relu is fmax: an E4M3 NaN code in a key or in one head's query makes
    that (key, head) product NaN, which contributes 0."""
    rng = np.random.default_rng(5)
    n, H, bs = 64, 16, 16
    keys = rng.integers(0, 256, size=(n, D), dtype=np.uint8)
    keys[(keys & 0x7F) == 0x7F] = 0
    keys[3, 10] = 0x7F                 # NaN code in key 3
    scales = rng.uniform(0.1, 1.0, size=n).astype(np.float32)
    q = rng.integers(0, 256, size=(1, H, D), dtype=np.uint8)
    q[(q & 0x7F) == 0x7F] = 0
    w = rng.standard_normal((1, H)).astype(np.float32)
    pages = page_layout(keys, scales, bs)
    bt = np.arange(pages.shape[0], dtype=np.int32)[None, :]
    base = oracle.fp8_paged_mqa_logits(q, pages, bs, w, np.array([n]), bt, n)
    assert np.isfinite(base[0]).all() and base[0, 3] == 0.0     # every head's product with key 3 dropped
    q2 = q.copy()
    q2[0, 5, 7] = 0xFF                 # NaN code in head 5
    got = oracle.fp8_paged_mqa_logits(q2, pages, bs, w, np.array([n]), bt, n)
    w5 = w.copy()
    w5[0, 5] = 0.0                     # head 5 removed instead
    want = oracle.fp8_paged_mqa_logits(q, pages, bs, w5, np.array([n]), bt, n)
    assert np.array_equal(got, want)
