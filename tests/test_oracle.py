"""Pins the CPU oracle against what fixes it independently of the oracle itself:
the reference's published known answers, exact rational arithmetic, closed
forms, independent formulations and mathematical invariants.  CPU only."""
import random
from fractions import Fraction

import numpy as np
import pytest

# num_tokens_post_padded known answers published by the reference for its
# GPU correctness run (docs/measurements.json:99-1444, 168 cases over
# B in {1, 2, 4, 8} x 7 patterns x 2 dtypes x 3 warp counts; patterns from
# benchmarks/moe_align.py:49-55 driven by random.Random(37)).
POSTPAD_KAT = {
    1: {"distinct": 64, "shared_top8": 64, "random_top8": 64, "all_one_expert": 8,
        "seven_experts": 56, "invalid_mixed": 40, "all_invalid": 0},
    2: {"distinct": 128, "shared_top8": 64, "random_top8": 128, "all_one_expert": 16,
        "seven_experts": 56, "invalid_mixed": 64, "all_invalid": 0},
    4: {"distinct": 256, "shared_top8": 64, "random_top8": 240, "all_one_expert": 32,
        "seven_experts": 56, "invalid_mixed": 80, "all_invalid": 0},
    8: {"distinct": 512, "shared_top8": 64, "random_top8": 488, "all_one_expert": 64,
        "seven_experts": 112, "invalid_mixed": 88, "all_invalid": 0},
}


# ---------------------------------------------------------------- MoE align

def numpy_align(flat):
    """Third formulation: stable argsort by expert (the shape of
    benchmarks/moe_align.py:70-92), independent of both C routines."""
    flat = np.asarray(flat, dtype=np.int64)
    R = flat.size
    key = np.where((flat >= 0) & (flat < 288), flat, 288)
    counts = np.bincount(key, minlength=289)[:288]
    padded = (counts + 7) // 8 * 8
    start = np.cumsum(padded) - padded
    first = np.cumsum(counts) - counts
    order = np.argsort(key, kind="stable")
    sorted_ids = np.full(R * 8, R, dtype=np.int32)
    experts = np.full(R, -1, dtype=np.int32)
    for pos, route in enumerate(order):
        e = key[route]
        if e == 288:
            continue
        rank = pos - first[e]
        sorted_ids[start[e] + rank] = route
        if rank % 8 == 0:
            experts[(start[e] + rank) // 8] = e
    return sorted_ids, experts, np.array([padded.sum()], dtype=np.int32)


def test_moe_postpad_known_answers(oracle):
    rng = random.Random(37)
    for batch in (1, 2, 4, 8):
        pats = oracle.moe_patterns(batch, rng)
        got = {name: int(oracle.moe_align(flat)[2][0]) for name, flat in pats.items()}
        assert got == POSTPAD_KAT[batch], batch


def test_moe_sweep_856_cases(oracle):
    """benchmarks/moe_align.py:58-67: 8 batches x (7 patterns + 100 random)."""
    rng = random.Random(37)
    cases = 0
    for batch in range(1, 9):
        pats = list(oracle.moe_patterns(batch, rng).values())
        pats += [[rng.randrange(-2, 292) for _ in range(batch * 8)] for _ in range(100)]
        for flat in pats:
            a = oracle.moe_align(flat)
            b = oracle.moe_align(flat, pairwise=True)
            c = numpy_align(flat)
            for x, y, z in zip(a, b, c):
                assert np.array_equal(x, y) and np.array_equal(x, z), (batch, flat)
            cases += 1
    assert cases == 856


def test_moe_closed_forms(oracle):
    # one token, 8 distinct experts in descending order: sorted by expert,
    # each expert alone in a padded block of 8
    flat = [7, 6, 5, 4, 3, 2, 1, 0]
    s, e, p = oracle.moe_align(flat)
    assert p[0] == 64
    assert list(e) == list(range(8))
    for blk in range(8):
        assert s[8 * blk] == 7 - blk and all(s[8 * blk + 1: 8 * blk + 8] == 8)
    # all invalid: nothing placed
    s, e, p = oracle.moe_align([-1, 288, 1 << 40, -(1 << 40)] * 2)
    assert p[0] == 0 and all(s == 8) and all(e == -1)
    # a 64-bit id that aliases a valid expert in its low 32 bits is invalid
    s, e, p = oracle.moe_align([(1 << 32) + 5] + [5] * 7)
    assert p[0] == 8 and list(s[:8]) == [1, 2, 3, 4, 5, 6, 7, 8] and e[0] == 5


# ---------------------------------------------------------------- store_int8

def exact_row(x_u16):
    """528-byte row by exact rational arithmetic (kernels/titan_kv.py:15-21):
    fp32 s = RN(amax / 127) clamped to fp32(1e-12), code = round-half-even of
    RN32(x / s), clamped to +-127."""
    import struct
    xs = [Fraction(struct.unpack("<f", struct.pack("<I", int(h) << 16))[0]) for h in x_u16]
    amax = max(abs(v) for v in xs)

    def rn32_exact(fr):
        # correctly rounded binary32 of a rational (float(fr) rounds to double
        # first; guard against double rounding by checking the neighbours)
        f = np.float32(float(fr))
        best = Fraction(float(f))
        for cand in (np.nextafter(f, np.float32(np.inf)), np.nextafter(f, np.float32(-np.inf))):
            c = Fraction(float(cand))
            d0, d1 = abs(best - fr), abs(c - fr)
            if d1 < d0 or (d1 == d0 and (int(np.float32(cand).view(np.uint32)) & 1) == 0):
                best = c
        return best

    s = rn32_exact(amax / 127)
    tiny = Fraction(float(np.float32(1e-12)))
    if not s > tiny:
        s = tiny
    codes = []
    for v in xs:
        qf = rn32_exact(v / s)
        fl = qf.numerator // qf.denominator
        rem = qf - fl
        q = fl + 1 if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1) else fl
        q = max(-127, min(127, q))
        codes.append(q & 0xFF)
    out = bytes(codes) + struct.pack("<f", float(s)) + bytes(12)
    return np.frombuffer(out, dtype=np.uint8)


def _bf16(vals):
    from oracle import f32_to_bf16
    return f32_to_bf16(np.asarray(vals, dtype=np.float32))


def test_store_int8_against_exact_rationals(oracle):
    rng = np.random.default_rng(20260910)
    rows = [rng.standard_normal(512).astype(np.float32) for _ in range(6)]
    rows.append(rng.standard_t(3, 512).astype(np.float32) * 0.5)
    rows.append(np.zeros(512, np.float32))                       # all-zero row
    ties = np.zeros(512, np.float32)
    ties[0] = 127.0                                              # s == 1 exactly
    ties[1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5]  # half-way cases
    rows.append(ties)
    rows.append(np.full(512, 1e-11, np.float32))                 # below the 1e-12 clamp * 127
    rows.append(np.full(512, 3e38, np.float32) * np.where(np.arange(512) % 2, 1, -1))
    x = np.stack([_bf16(r) for r in rows])
    got = oracle.quantize_rows(x)
    for i in range(len(rows)):
        want = exact_row(x[i])
        assert np.array_equal(got[i], want), i
    # closed forms
    t = got[8, :9].view(np.int8)
    assert list(t) == [127, 0, 2, 2, 0, -2, -2, 126, -126]   # ties to even
    assert got[7, :512].max() == 0 and oracle.row_scales(got[7:8])[0] == np.float32(1e-12)
    for i in range(7):
        codes = got[i, :512].view(np.int8).astype(int)
        amax_pos = np.argmax(np.abs(oracle.bf16_to_f32(x[i])))
        assert abs(codes[amax_pos]) == 127
        assert np.all(got[i, 516:] == 0)


def test_store_int8_layout_and_negative_slot(oracle):
    rng = np.random.default_rng(1)
    x = _bf16(rng.standard_normal((40, 512)))
    nb, block = 3, 16
    cache = np.full((nb, block, 528), 0xAB, dtype=np.uint8)
    slots = np.array([5, -1, 47, 0, 16, -7] + list(range(17, 45)), dtype=np.int64)[:40]
    oracle.store_int8(x[:slots.size], cache, slots)
    flat = cache.reshape(-1, 528)
    rows = oracle.quantize_rows(x)
    written = set()
    for i, s in enumerate(slots):
        if s >= 0:
            assert np.array_equal(flat[s], rows[i])
            written.add(int(s))
    for s in range(nb * block):
        if s not in written:
            assert np.all(flat[s] == 0xAB)
    # a padded block stride (e.g. a page with trailing bytes) is honoured
    big = np.zeros((2, 4 * 528 + 64), dtype=np.uint8)
    view = np.lib.stride_tricks.as_strided(big, shape=(2, 4, 528), strides=(4 * 528 + 64, 528, 1))
    oracle.store_int8(x[:8], view, np.arange(8))
    assert np.array_equal(big[1, :528], rows[4]) and np.all(big[:, 4 * 528:] == 0)


# ---------------------------------------------------------------- sparse MLA

def numpy_attention(q_u16, rows, idx, sm_scale):
    """Textbook float64 softmax attention in numpy over dequantised rows."""
    from oracle import bf16_to_f32, dequantize
    q = bf16_to_f32(q_u16).astype(np.float64)
    kvf = dequantize(rows)
    T, H, _ = q.shape
    out = np.zeros((T, H, 512))
    for t in range(T):
        ids = idx[t]
        ok = (ids >= 0) & (ids < rows.shape[0])
        if not ok.any():
            continue
        k = kvf[ids[ok]]
        logits = q[t] @ k.T * sm_scale
        logits -= logits.max(axis=1, keepdims=True)
        w = np.exp(logits)
        w /= w.sum(axis=1, keepdims=True)
        out[t] = w @ k
    return out


def _mla_case(oracle, T=2, H=16, seq=4096, topk=256, pad=32, seed=3, dist="normal"):
    rng = np.random.default_rng(seed)
    lat = rng.standard_normal((seq, 512)) if dist == "normal" else rng.standard_t(3, (seq, 512)) * 0.5
    rows = oracle.quantize_rows(_bf16(lat))
    q = _bf16(rng.standard_normal((T, H, 512)))
    idx = rng.integers(0, seq, size=(T, topk)).astype(np.int32)
    if pad:
        idx[:, topk - pad:] = -1
    return q, rows, idx


def test_mla_f64_implementations_agree(oracle):
    q, rows, idx = _mla_case(oracle)
    idx[0, 3] = rows.shape[0] + 5          # positive out-of-range index
    a = oracle.sparse_mla_f64(q, rows, idx, 512 ** -0.5)
    b = numpy_attention(q, rows, idx, 512 ** -0.5)
    assert np.max(np.abs(a - b)) < 1e-12


@pytest.mark.parametrize("splits", [1, 4, 8, 32])
def test_mla_faithful_vs_textbook(oracle, splits):
    from oracle import bf16_to_f32
    q, rows, idx = _mla_case(oracle, topk=512, pad=64)
    ref = oracle.sparse_mla_f64(q, rows, idx, 512 ** -0.5)
    out = bf16_to_f32(oracle.sparse_mla(q, rows, idx, 512 ** -0.5, n_splits=splits))
    err = np.abs(out - ref)
    assert err.max() < 2e-2 and err.mean() < 2e-3
    nmse = ((out - ref) ** 2).sum() / (ref ** 2).sum()
    assert nmse < 1e-4


@pytest.mark.parametrize("splits", [1, 8])
@pytest.mark.parametrize("groups,block_n,lazy", [(2, 32, 0.0), (4, 32, 0.0), (4, 16, 8.0)])
def test_mla_key_groups_match_single_stream(oracle, splits, groups, block_n, lazy):
    """Tiles dealt to several online-softmax streams (the HIP kernel's key
    groups; also with a lazily moved max) merged at the end agree with the
    reference's single stream, and with textbook attention, to the output
    bar."""
    from oracle import bf16_to_f32
    for dist in ("normal", "t3"):
        q, rows, idx = _mla_case(oracle, T=3, topk=2176, pad=128, dist=dist, seed=9)
        one = bf16_to_f32(oracle.sparse_mla(q, rows, idx, 512 ** -0.5, n_splits=splits))
        two = bf16_to_f32(oracle.sparse_mla(q, rows, idx, 512 ** -0.5, n_splits=splits, groups=groups,
                                            block_n=block_n, lazy=lazy))
        err = np.abs(one - two)
        ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(one), 2.0 ** -126))) - 7)
        assert np.all(err <= np.maximum(2e-2, ulp)) and err.mean() < 2e-4, dist
        ref = oracle.sparse_mla_f64(q, rows, idx, 512 ** -0.5)
        nmse = ((two - ref) ** 2).sum() / (ref ** 2).sum()
        assert nmse < 1e-4, dist


def test_literal_bar_breaks_under_reordering(oracle):
    """Why the GPU bar lets rare elements with |ref| >= 4 differ by one bf16
    ulp instead of 2e-2: the reference's own arithmetic, run in one
    online-softmax stream and dealt to two streams (the same products and
    rounding points, only the fp32 summation order differs), already gives
    such elements on heavy-tailed data.  128 queries over a 16384-row
    Student-t(3) x 0.5 cache, 2176 uniform indices (numpy seed 1)."""
    from oracle import bf16_to_f32, f32_to_bf16
    rng = np.random.default_rng(1)
    n = 16384
    z = rng.standard_normal((n, 512), dtype=np.float32)
    chi = sum(rng.standard_normal((n, 512), dtype=np.float32) ** 2 for _ in range(3))
    rows = oracle.quantize_rows(f32_to_bf16((z / np.sqrt(chi / 3) * 0.5).astype(np.float32)),
                                nthreads=oracle.default_threads())
    q = f32_to_bf16(rng.standard_normal((128, 16, 512)).astype(np.float32))
    idx = rng.integers(0, n, size=(128, 1, 2176)).astype(np.int32)
    th = oracle.default_threads()
    one = bf16_to_f32(oracle.sparse_mla(q, rows, idx, 512 ** -0.5, nthreads=th))
    two = bf16_to_f32(oracle.sparse_mla(q, rows, idx, 512 ** -0.5, nthreads=th, groups=2))
    err = np.abs(one - two)
    over = err > 2e-2
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(one), 2.0 ** -126))) - 7)
    assert over.sum() >= 1                                   # the literal bar fails ...
    assert np.all(np.abs(one[over]) >= 4)                    # ... only where a bf16 ulp exceeds 2e-2
    assert np.all(err[over] == ulp[over])                    # ... by exactly one bf16 ulp
    assert over.sum() <= err.size // 100000 + 2 and err.mean() < 2e-4


def test_mla_wrong_scale_is_caught(oracle):
    """A plausible slip (sm_scale not applied / log2e dropped) fails the bar."""
    from oracle import bf16_to_f32
    q, rows, idx = _mla_case(oracle, topk=512, pad=64)
    ref = oracle.sparse_mla_f64(q, rows, idx, 512 ** -0.5)
    bad = bf16_to_f32(oracle.sparse_mla(q, rows, idx, 512 ** -0.5 / 1.4426950408889634))
    err = np.abs(bad - ref)
    assert not (err.max() < 2e-2 and err.mean() < 2e-3)


def test_mla_invariants(oracle):
    from oracle import bf16_to_f32, dequantize
    q, rows, idx = _mla_case(oracle, T=1, topk=256, pad=0, seed=5)
    base = bf16_to_f32(oracle.sparse_mla(q, rows, idx, 512 ** -0.5, n_splits=1))
    # split-count invariance
    for s in (2, 4, 8, 16, 100):
        o = bf16_to_f32(oracle.sparse_mla(q, rows, idx, 512 ** -0.5, n_splits=s))
        assert np.max(np.abs(o - base)) < 4e-3, s
    # permutation invariance
    perm = np.random.default_rng(0).permutation(idx.shape[1])
    o = bf16_to_f32(oracle.sparse_mla(q, rows, idx[:, perm], 512 ** -0.5))
    assert np.max(np.abs(o - base)) < 4e-3
    # all masked -> exactly zero (tests/verify_mla.py:91-93)
    blank = oracle.sparse_mla(q, rows, np.full_like(idx, -1), 512 ** -0.5, n_splits=4)
    assert np.all(blank == 0)
    oob = oracle.sparse_mla(q, rows, np.full_like(idx, rows.shape[0]), 512 ** -0.5)
    assert np.all(oob == 0)
    # a single valid index -> that dequantised row (to bf16 rounding of p*scale)
    one = np.full_like(idx, -1)
    one[0, 77] = 1234
    o = bf16_to_f32(oracle.sparse_mla(q, rows, one, 512 ** -0.5))
    want = dequantize(rows[1234:1235])[0]
    assert np.max(np.abs(o[0] - want[None, :])) <= 0.02 * np.abs(want).max()
    # q = 0 -> the mean of the valid rows
    qz = np.zeros_like(q)
    o = bf16_to_f32(oracle.sparse_mla(qz, rows, idx, 512 ** -0.5))
    mean = dequantize(rows[idx[0]]).mean(axis=0)
    assert np.max(np.abs(o[0] - mean[None, :])) < 2e-3


def test_split_heuristic_hand_table(oracle):
    """kernels/titan_mla.py:432-449 at the reference's 70 SMs."""
    assert [oracle.choose_num_kv_splits(t, 1, 2176, 70) for t in (1, 6, 8, 2048)] == [32, 8, 8, 1]
    assert oracle.choose_num_kv_splits(0, 1, 2176, 70) == 1
    assert oracle.choose_num_kv_splits(1, 1, 96, 70) == 1


# ---- request-relative index conversion (vLLM helper; parity with vLLM unpinned) ----

def _paged_case(rng, num_reqs=3, block_size=16, page_rows=19, max_blocks=6, num_blocks=24):
    """Physical pages of page_rows rows (only the first block_size hold
    tokens), a block table of distinct pages per request."""
    perm = rng.permutation(num_blocks)[: num_reqs * max_blocks].reshape(num_reqs, max_blocks)
    return perm.astype(np.int32), block_size, page_rows, num_blocks


def test_convert_identity_table(oracle):
    """One request whose table is 0, 1, 2, ... and unpadded pages: a position
    maps to itself; past the table, or negative, to -1."""
    bt = np.arange(5, dtype=np.int32)[None, :]
    p = np.array([[0, 1, 15, 16, 79, 80, 81, -1, -7, 1000]])
    out = oracle.convert_req_index(np.array([0]), bt, p, 16)
    assert out.tolist() == [[0, 1, 15, 16, 79, -1, -1, -1, -1, -1]]


def test_convert_decomposes_into_page_and_offset(oracle):
    rng = np.random.default_rng(4)
    bt, bs, pr, nb = _paged_case(rng)
    req = np.array([2, 0, 1, 7, -1])
    p = rng.integers(-3, bt.shape[1] * bs + 9, size=(5, 64))
    out = oracle.convert_req_index(req, bt, p, bs, pr)
    for t in range(5):
        for k in range(64):
            valid = 0 <= req[t] < bt.shape[0] and 0 <= p[t, k] < bt.shape[1] * bs
            if not valid:
                assert out[t, k] == -1
            else:
                page, off = divmod(int(out[t, k]), pr)
                assert page == bt[req[t], p[t, k] // bs] and off == p[t, k] % bs < bs


def test_convert_wraps_like_int32(oracle):
    bt = np.array([[2 ** 30 + 3]], dtype=np.int32)
    out = oracle.convert_req_index(np.array([0]), bt, np.array([[5]]), 8, 8)
    assert out[0, 0] == np.int32(np.uint32(((2 ** 30 + 3) * 8 + 5) % 2 ** 32).view(np.int32))


@pytest.mark.parametrize("page_rows", [16, 19])
def test_paged_attention_equals_logical_cache(oracle, page_rows):
    """Attention through converted indices over the flat paged rows equals
    attention over each request's logically ordered cache (its pages
    concatenated in block-table order) indexed by the raw positions; a
    slip (page stride taken as block_size with padded pages, or div / mod
    swapped) gathers other rows and fails."""
    from oracle import bf16_to_f32
    rng = np.random.default_rng(11)
    bt, bs, _, nb = _paged_case(rng, page_rows=page_rows)
    pr = page_rows
    lat = rng.standard_normal((nb * pr, 512))
    flat = oracle.quantize_rows(_bf16(lat))
    T, topk = 4, 128
    req = np.array([1, 0, 2, 1])
    q = _bf16(rng.standard_normal((T, 16, 512)))
    p = rng.integers(0, bt.shape[1] * bs, size=(T, topk)).astype(np.int32)
    p[:, -16:] = -1
    conv = oracle.convert_req_index(req, bt, p, bs, pr)
    via_pages = bf16_to_f32(oracle.sparse_mla(q, flat, conv, 512 ** -0.5, n_splits=2))
    for t in range(T):
        logical = np.concatenate([flat[bt[req[t], j] * pr: bt[req[t], j] * pr + bs] for j in range(bt.shape[1])])
        one = bf16_to_f32(oracle.sparse_mla(q[t:t + 1], logical, p[t:t + 1], 512 ** -0.5, n_splits=2))
        assert np.array_equal(one[0], via_pages[t]), t
    if pr != bs:
        slip = oracle.convert_req_index(req, bt, p, bs, bs)
        bad = bf16_to_f32(oracle.sparse_mla(q, flat, slip, 512 ** -0.5, n_splits=2))
        assert not np.array_equal(bad, via_pages)
    swapped = np.where(p >= 0, (p % bs) * bs + p // bs, -1)   # div / mod swapped
    bad2 = bf16_to_f32(oracle.sparse_mla(q, flat, oracle.convert_req_index(req, bt, swapped, bs, pr), 512 ** -0.5,
                                         n_splits=2))
    assert not np.array_equal(bad2, via_pages)


# ---- kpool expansion (the indexer's last step) ----

def test_expand_pools_closed_forms(oracle):
    out = oracle.expand_pools(np.array([[2, -1, 0]]), np.array([11]), 4)
    assert out.tolist() == [[8, 9, 10, 11, -1, -1, -1, -1, 0, 1, 2, 3, 8, 9, 10]]
    out = oracle.expand_pools(np.array([[5, 1]]), np.array([8]), 4, out_cols=12)
    assert out.tolist() == [[20, 21, 22, 23, 4, 5, 6, 7, -1, -1, -1, -1]]   # 8 % 4 == 0: empty tail
    assert oracle.expand_pools(np.array([[3]]), None, 1).tolist() == [[3]]
    assert oracle.expand_pools(np.array([[7, 2]]), np.array([100]), 1).tolist() == [[7, 2]]  # pool 1: no tail slots


def test_expand_pools_set_formulation(oracle):
    """The multiset of valid positions equals the union of each valid pool's
    tokens and the tail tokens [len // P * P, len), and every slot's position
    lies in its own pool (or the tail range)."""
    rng = np.random.default_rng(8)
    for P in (1, 2, 4, 5):
        pools = rng.integers(-2, 300, size=(6, 37))
        lens = rng.integers(0, 1300, size=6)
        out = oracle.expand_pools(pools, lens, P, out_cols=37 * P + P - 1 + 9)
        for r in range(6):
            want = sorted([int(p) * P + o for p in pools[r] if p >= 0 for o in range(P)] +
                          list(range(lens[r] // P * P, lens[r])))
            got = out[r]
            assert sorted(int(v) for v in got if v >= 0) == want
            for k, v in enumerate(got[: 37 * P]):
                assert v == -1 or v // P == pools[r, k // P]
            assert np.all(got[37 * P + P - 1:] == -1)
