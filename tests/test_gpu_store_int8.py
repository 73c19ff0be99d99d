"""GPU parity of store_int8 (HIP) against the CPU oracle: bit-exact rows."""
import numpy as np
import pytest
import torch

import workloads as W
from conftest import log_case
from parity_log import record_exact

pytestmark = pytest.mark.gpu


def u16(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def u8(t):
    return t.contiguous().view(torch.uint8).cpu().numpy()


def test_writer_small_bit_exact(cuda, oracle):
    from titan_kv import store_int8
    log_case("store_int8 writer_small 16384 rows")
    w = W.writer_small(cuda, seed=W.SEED_FIXTURE)
    store_int8(w["x"], w["cache"], w["slots"])
    torch.cuda.synchronize()
    got = u8(w["cache"]).reshape(-1, 528)
    want = oracle.quantize_rows(u16(w["x"]), nthreads=oracle.default_threads())
    record_exact("rows16384_b1", "store_int8 rows (bytes)", np.count_nonzero(got != want), got.size)
    assert np.array_equal(got, want)


def test_covering_set_bit_exact(cuda, oracle):
    """Every bf16 x with |x| <= amax for all 128 mantissas of amax in [1, 2),
    plus row maxima in the 1e-12 clamp range, near the bf16 maximum and
    subnormal: the quotient domain up to a power-of-two scale."""
    from titan_kv import store_int8
    log_case("store_int8 covering set")
    rows = []
    for mant in range(128):
        a = 0x3F80 | mant                       # amax in [1, 2)
        xs = np.arange(0, a + 1, dtype=np.uint16)
        xs = np.concatenate([xs, xs[1:] | 0x8000])
        for s in range(0, xs.size, 511):
            r = np.zeros(512, np.uint16)
            chunk = xs[s:s + 511]
            r[:chunk.size] = chunk
            r[511] = a
            rows.append(r)
    rng = np.random.default_rng(7)
    for a in (0x2D00, 0x2E8F, 0x0001, 0x007F, 0x0080, 0x7F7F, 0x7F00, 0x4300):
        for _ in range(4):
            m = rng.integers(0, a + 1, 511).astype(np.uint16)
            m |= (rng.integers(0, 2, 511).astype(np.uint16) << 15)
            rows.append(np.concatenate([m, np.array([a | 0x8000], np.uint16)]))
    x = np.stack(rows)
    n = x.shape[0]
    xt = torch.from_numpy(x.view(np.int16)).to(cuda).view(torch.bfloat16)
    cache = torch.zeros(n, 1, 528, device=cuda, dtype=torch.int8)
    store_int8(xt, cache, torch.arange(n, device=cuda))
    torch.cuda.synchronize()
    got = u8(cache).reshape(n, 528)
    want = oracle.quantize_rows(x, nthreads=oracle.default_threads())
    bad = np.nonzero((got != want).any(axis=1))[0]
    assert bad.size == 0, f"{bad.size} rows differ, first {bad[:5]}"


def test_slots_layouts_and_guards(cuda, oracle):
    from titan_kv import store_int8
    log_case("store_int8 slot layouts")
    g = W.gen(cuda, 11)
    x = W.latents(600, cuda, g)
    rows = oracle.quantize_rows(u16(x))
    # scattered int32 slots with negatives and out-of-capacity entries
    cache = torch.full((4, 256, 528), 0x55, device=cuda, dtype=torch.int8)
    perm = torch.randperm(1024, generator=g, device=cuda)[:600].to(torch.int32)
    perm[::7] = -1
    perm[5] = 1024          # == capacity: skipped
    perm[6] = 1 << 30       # far beyond: skipped
    store_int8(x, cache, perm)
    torch.cuda.synchronize()
    flat = u8(cache).reshape(-1, 528)
    p = perm.cpu().numpy()
    touched = np.zeros(1024, bool)
    for i, s in enumerate(p):
        if 0 <= s < 1024:
            assert np.array_equal(flat[s], rows[i]), i
            touched[s] = True
    assert np.all(flat[~touched] == 0x55)
    # strided x (row stride 640 elements, 16-B aligned) and an unaligned view
    wide = torch.zeros(600, 640, device=cuda, dtype=torch.bfloat16)
    wide[:, :512] = x
    for xv, tag in ((wide[:, :512], "aligned stride"), (wide[:, 3:515], "unaligned view")):
        c2 = torch.zeros(3, 256, 528, device=cuda, dtype=torch.uint8)
        store_int8(xv, c2, torch.arange(600, device=cuda))
        torch.cuda.synchronize()
        want = oracle.quantize_rows(u16(xv))
        assert np.array_equal(u8(c2).reshape(-1, 528)[:600], want), tag
    # padded block stride: a page of 256 rows followed by 4096 spare bytes
    pages = torch.zeros(3, 256 * 528 + 4096, device=cuda, dtype=torch.uint8)
    view = pages[:, :256 * 528].view(3, 256, 528)
    store_int8(x, view, torch.arange(600, device=cuda, dtype=torch.int64))
    torch.cuda.synchronize()
    assert np.array_equal(u8(view).reshape(-1, 528)[:600], rows)
    assert int(pages[:, 256 * 528:].abs().sum().item()) == 0
    # negative slot leaves the cache untouched (tests/verify_mla.py:67-69)
    before = cache.clone()
    store_int8(x[:1], cache, torch.tensor([-1], device=cuda))
    torch.cuda.synchronize()
    assert torch.equal(before, cache)


def test_reference_fixture_properties(cuda):
    """The reference's own checks on its fixture (tests/verify_mla.py:30-66):
    columns scaled by 0.05 and 8, row 0 zero; scale within rtol 1e-6 of
    clamp(amax)/127, |int error| <= 1 against torch.round, zero padding,
    quantisation NMSE < 3e-4."""
    from titan_kv import store_int8
    log_case("store_int8 reference fixture properties")
    g = W.gen(cuda, W.SEED_FIXTURE)
    n = 65536
    orig = torch.randn(n, 512, device=cuda, dtype=torch.bfloat16, generator=g)
    orig[:, :128] *= 0.05
    orig[:, 256:384] *= 8
    orig[0] = 0
    cache = torch.zeros(n // 256, 256, 528, device=cuda, dtype=torch.int8)
    store_int8(orig, cache, torch.arange(n, device=cuda, dtype=torch.int64))
    rows = cache.view(n, 528)
    vals = orig.float()
    scales = rows[:, 512:516].contiguous().view(torch.float32)
    expected = vals.abs().amax(dim=1, keepdim=True).clamp_min(127e-12) / 127
    torch.testing.assert_close(scales, expected, rtol=1e-6, atol=1e-12)
    ints = rows[:, :512].float()
    assert (ints - torch.round(vals / expected).clamp(-127, 127)).abs().max().item() <= 1
    deq = (ints * scales).to(torch.bfloat16).float()
    nmse = ((deq - vals) ** 2).sum().item() / (vals ** 2).sum().item()
    assert nmse < 3e-4
    assert bool((rows[:, 516:] == 0).all())


@pytest.mark.slow
def test_full_context_writer_bit_exact(cuda, oracle):
    """262144-row cache (the decode configurations' size), N(0,1) and
    Student-t latents."""
    from titan_kv import store_int8
    for dist in ("normal", "t3"):
        log_case("store_int8 262144 rows", dist)
        g, x, cache, slots = W.decode_cache(cuda, seed=W.SEED_BENCH, dist=dist)
        store_int8(x, cache, slots)
        torch.cuda.synchronize()
        got = u8(cache).reshape(-1, 528)
        want = oracle.quantize_rows(u16(x), nthreads=oracle.default_threads())
        record_exact("rows262144_normal_b1" if dist == "normal" else "rows262144_t3_b8", "store_int8 rows (bytes)",
                     np.count_nonzero(got != want), got.size)
        assert np.array_equal(got, want), dist
        del x, cache
        torch.cuda.empty_cache()


@pytest.mark.slow
def test_prefill_scattered_writer_full_size(cuda, oracle):
    """The prefill-shaped call's write: 2048 new N(0,1) rows into a random
    permutation of the slots of a [1024, 256, 528] cache that already holds
    262144 rows; every written row bit-exact, every other row untouched."""
    from titan_kv import store_int8
    log_case("store_int8 2048 rows -> randperm slots of a 262144-row cache")
    g = W.gen(cuda, W.SEED_BENCH + 5)
    old = torch.randint(-128, 128, (1024, 256, 528), generator=g, device=cuda, dtype=torch.int8)
    cache = old.clone()
    _, _, new_rows, slots = W.prefill_inputs(cuda, g)
    assert slots.dtype == torch.int64 and slots.numel() == 2048
    store_int8(new_rows, cache, slots)
    torch.cuda.synchronize()
    flat = u8(cache).reshape(-1, 528)
    was = u8(old).reshape(-1, 528)
    s = slots.cpu().numpy()
    want = oracle.quantize_rows(u16(new_rows), nthreads=oracle.default_threads())
    untouched = np.ones(flat.shape[0], bool)
    untouched[s] = False
    record_exact("prefill_t2048", "store_int8 scattered rows (bytes)", np.count_nonzero(flat[s] != want), want.size)
    record_exact("prefill_t2048", "rows not written (bytes changed)", np.count_nonzero(flat[untouched] != was[untouched]),
                 flat[untouched].size)
    assert np.array_equal(flat[s], want)
    assert np.array_equal(flat[untouched], was[untouched])
