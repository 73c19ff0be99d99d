"""Pins the oracle of the W4A16 group-32 MoE layer (oracle.moe_w4a16 and its
packing helpers) against what fixes it without the oracle: bit-level brute
force of the packing, closed forms built from single codes and uniform
weights (every index of the layer -- expert, gate/up half, output row, input
feature, scale group, route slot -- moves a known value to a known place),
the SiLU clamp, invariants over the routes, and an independent torch
formulation.  CPU only."""
import math

import numpy as np
import pytest


def bf16(v):
    import oracle
    return oracle.f32_to_bf16(np.asarray(v, dtype=np.float32))


def f32(u):
    import oracle
    return oracle.bf16_to_f32(u)


def rbf16(v):
    """Round a float to bf16 and back (float)."""
    return float(f32(bf16(np.float32(v))).reshape(-1)[0])


def layer(oracle, E, N, K, codes13, sc13, codes2, sc2):
    return (oracle.pack_w4(codes13), bf16(sc13), oracle.pack_w4(codes2), bf16(sc2))


# ---------------------------------------------------------------- packing

def test_unpack_matches_bit_extraction(oracle):
    rng = np.random.default_rng(1)
    words = rng.integers(-2**31, 2**31, size=(3, 5, 4), dtype=np.int64).astype(np.int32)
    codes = oracle.unpack_w4(words)
    assert codes.shape == (3, 5, 32)
    for idx in np.ndindex(3, 5, 32):
        w = int(words[idx[0], idx[1], idx[2] // 8]) & 0xFFFFFFFF
        assert codes[idx] == (w >> (4 * (idx[2] % 8))) & 0xF
    assert np.array_equal(oracle.pack_w4(codes), words)


def test_repack_layout_brute_force(oracle):
    rng = np.random.default_rng(2)
    codes = rng.integers(0, 16, size=(3, 48, 384), dtype=np.uint8)
    tiles = oracle.repack_w4a16(oracle.pack_w4(codes)).view(np.uint32)
    assert tiles.shape == (3, 3, 3, 64, 4)
    for e in range(3):
        for nt in range(3):
            for c in range(3):
                for lane in range(64):
                    for i in range(4):
                        word = int(tiles[e, nt, c, lane, i])
                        for j in range(8):
                            k = 32 * (4 * c + i) + 8 * (lane // 16) + j
                            bit = 4 * (j // 2) + 16 * (j % 2)
                            assert (word >> bit) & 0xF == codes[e, 16 * nt + lane % 16, k]


def test_scale_repack_layout_brute_force(oracle):
    rng = np.random.default_rng(7)
    sc = rng.integers(0, 2**16, size=(2, 48, 12), dtype=np.uint16)
    t = oracle.repack_w4a16_scales(sc)
    assert t.shape == (2, 3, 3, 16, 4)
    for e, nt, c, r, g in np.ndindex(*t.shape):
        assert t[e, nt, c, r, g] == sc[e, 16 * nt + r, 4 * c + g]


def test_magic_decode_is_code_plus_128():
    # (word >> 4j) & 0x000F000F | 0x43004300 read as two bf16 = 128 + code
    for code in range(16):
        bits = np.array([0x4300 | code], dtype=np.uint16)
        assert float((bits.astype(np.uint32) << 16).view(np.float32)[0]) == 128 + code
    assert float((np.array([0xC308], np.uint32) << 16).view(np.float32)[0]) == -136.0


# ---------------------------------------------------------------- closed forms

def test_uniform_weights_closed_form(oracle):
    E, N, K, T = 3, 32, 256, 2
    s13, s2 = 2.0 ** -9, 2.0 ** -6
    codes13 = np.full((E, 2 * N, K), 9, np.uint8)        # W13 = +s13 everywhere
    codes2 = np.full((E, K, N), 9, np.uint8)             # W2 = +s2 everywhere
    w13, q13, w2, q2 = layer(oracle, E, N, K, codes13, np.full((E, 2 * N, K // 32), s13),
                             codes2, np.full((E, K, N // 32), s2))
    x = np.zeros((T, K), np.float32)
    x[0, :] = 1.0                                  # sum 256
    x[1, ::2] = -0.5                               # sum -64
    ids = np.array([[0, 1, 2, 0, 1, 2, 0, 1], [2, 2, 2, 2, 2, 2, 2, 2]], np.int32)
    tw = np.array([[0.5, 0.25, 0.125, 0.0625, 0.03125, 0.015625, 0.0078125, 0.0078125],
                   [1, 0, 0, 0, 0, 0, 0, 0]], np.float32)
    out, act = oracle.moe_w4a16(bf16(x), w13, q13, w2, q2, tw, ids, clamp_limit=10.0)
    for t in range(T):
        h = rbf16(s13 * float(x[t].sum()))       # every gate and up value
        g, u = min(h, 10.0), max(min(h, 10.0), -10.0)
        c2 = rbf16(np.float32(g) / (np.float32(1) + np.exp(np.float32(-g))) * np.float32(u))
        assert np.all(f32(act[8 * t:8 * t + 8]) == c2)
        y = np.float32(s2 * N * c2)              # exact: power-of-two scale, 32 equal terms
        total = np.float32(0)
        for j in range(8):
            total += np.float32(rbf16(tw[t, j] * y))
        assert np.all(f32(out[t]) == rbf16(total))


def test_single_codes_move_known_values(oracle):
    """Each expert gets one nonzero gate code, one nonzero up code and one
    nonzero down code at its own positions, with distinct scales per group:
    the output must be nonzero only at the expert's down row, with the value
    the three codes and their group scales fix."""
    rng = np.random.default_rng(3)
    E, N, K, T = 4, 64, 256, 1
    codes13 = np.full((E, 2 * N, K), 8, np.uint8)
    codes2 = np.full((E, K, N), 8, np.uint8)
    sc13 = rng.uniform(0.01, 0.05, size=(E, 2 * N, K // 32))
    sc2 = rng.uniform(0.01, 0.05, size=(E, K, N // 32))
    plan = {0: (5, 37, 200, 77), 1: (40, 3, 129, 250), 3: (63, 255, 0, 8)}   # n0, k_gate, k_up, k_out
    for e, (n0, kg, ku, ko) in plan.items():
        codes13[e, n0, kg] = 15          # gate weight +7 s
        codes13[e, N + n0, ku] = 0       # up weight -8 s
        codes2[e, ko, n0] = 12           # down weight +4 s
    w13, q13, w2, q2 = layer(oracle, E, N, K, codes13, sc13, codes2, sc2)
    x = rng.standard_normal((T, K)).astype(np.float32)
    xb = f32(bf16(x))
    ids = np.array([[0, 1, 3, -1, 288, 2**31 - 1, -7, 1000]], np.int64)
    tw = np.array([[0.5, 0.75, 1.25, 9, 9, 9, 9, 9]], np.float32)
    out, act = oracle.moe_w4a16(bf16(x), w13, q13, w2, q2, tw, ids, clamp_limit=None)
    want = np.zeros(K, np.float32)
    s = lambda a: float(f32(bf16(a)).reshape(-1)[0])
    for j, e in enumerate((0, 1, 3)):
        n0, kg, ku, ko = plan[e]
        g = rbf16(7 * s(sc13[e, n0, kg // 32]) * float(xb[0, kg]))
        u = rbf16(-8 * s(sc13[e, N + n0, ku // 32]) * float(xb[0, ku]))
        c2 = rbf16(np.float32(g) / (np.float32(1) + np.exp(np.float32(-g))) * np.float32(u))
        row = f32(act[j])
        assert row[n0] == c2 and np.count_nonzero(row) == (c2 != 0)
        y = np.float32(4 * s(sc2[e, ko, n0 // 32]) * c2)
        want[ko] += np.float32(rbf16(tw[0, j] * y))
    assert np.array_equal(f32(out[0]), f32(bf16(want)))
    assert np.count_nonzero(f32(out[0])) == 3


def test_clamp_limits_gate_and_up(oracle):
    E, N, K = 1, 32, 128
    codes13 = np.full((E, 2 * N, K), 9, np.uint8)
    codes2 = np.full((E, K, N), 9, np.uint8)
    w13, q13, w2, q2 = layer(oracle, E, N, K, codes13, np.full((E, 2 * N, 4), 0.25),
                             codes2, np.full((E, K, 1), 2.0 ** -5))
    ids = np.zeros((2, 8), np.int32)
    tw = np.zeros((2, 8), np.float32)
    tw[:, 0] = 1
    x = np.zeros((2, K), np.float32)
    x[0] = 1.0          # h = 32: gate -> 10, up -> 10
    x[1] = -1.0         # h = -32: gate stays -32, up -> -10
    _, act = oracle.moe_w4a16(bf16(x), w13, q13, w2, q2, tw, ids, clamp_limit=10.0)
    f = lambda g, u: rbf16(np.float32(g) / (np.float32(1) + np.exp(np.float32(-g))) * np.float32(u))
    assert np.all(f32(act[0]) == f(10.0, 10.0))
    assert np.all(f32(act[8]) == f(-32.0, -10.0))
    _, act_free = oracle.moe_w4a16(bf16(x), w13, q13, w2, q2, tw, ids, clamp_limit=None)
    assert np.all(f32(act_free[0]) == f(32.0, 32.0))
    assert np.all(f32(act_free[8]) == f(-32.0, -32.0))


# ---------------------------------------------------------------- invariants

def random_layer(oracle, rng, E=6, N=64, K=256):
    codes13 = rng.integers(0, 16, size=(E, 2 * N, K), dtype=np.uint8)
    codes2 = rng.integers(0, 16, size=(E, K, N), dtype=np.uint8)
    sc13 = rng.uniform(0.5, 1.5, size=(E, 2 * N, K // 32)) / (4.6 * math.sqrt(K))
    sc2 = rng.uniform(0.5, 1.5, size=(E, K, N // 32)) / (2.3 * math.sqrt(N))
    return layer(oracle, E, N, K, codes13, sc13, codes2, sc2)


def test_invalid_route_equals_zero_weight(oracle):
    rng = np.random.default_rng(4)
    E, N, K, T = 6, 64, 256, 3
    w = random_layer(oracle, rng, E, N, K)
    x = bf16(rng.standard_normal((T, K)))
    ids = rng.integers(0, E, size=(T, 8)).astype(np.int32)
    tw = rng.uniform(0, 1, size=(T, 8)).astype(np.float32)
    ids_bad, tw_zero = ids.copy(), tw.copy()
    ids_bad[:, [2, 5]] = [-1, E]
    tw_zero[:, [2, 5]] = 0
    a, _ = oracle.moe_w4a16(x, *w, tw, ids_bad)
    b, _ = oracle.moe_w4a16(x, *w, tw_zero, ids)
    assert np.array_equal(a, b)
    z, act = oracle.moe_w4a16(x, *w, tw, np.full((T, 8), -1, np.int32))
    assert not np.any(f32(z)) and not np.any(act)


def test_slot_order_only_changes_the_sum_order(oracle):
    rng = np.random.default_rng(5)
    E, N, K, T = 6, 64, 256, 2
    w = random_layer(oracle, rng, E, N, K)
    x = bf16(rng.standard_normal((T, K)))
    ids = rng.integers(0, E, size=(T, 8)).astype(np.int32)
    tw = rng.uniform(0, 1, size=(T, 8)).astype(np.float32)
    perm = rng.permutation(8)
    a, act_a = oracle.moe_w4a16(x, *w, tw, ids)
    b, act_b = oracle.moe_w4a16(x, *w, tw[:, perm], ids[:, perm])
    for t in range(T):
        assert np.array_equal(act_a[8 * t + perm], act_b[8 * t:8 * t + 8])
    d = np.abs(f32(a) - f32(b))
    assert d.max() <= 2.0 ** -7 * np.abs(f32(a)).max()


def test_matches_torch_formulation(oracle):
    """An independent formulation: torch unpacks with integer ops, dequantises
    with repeat_interleave, and uses F.silu / matmul in float64."""
    import torch
    import torch.nn.functional as F
    rng = np.random.default_rng(6)
    E, N, K, T = 5, 64, 256, 4
    w13, q13, w2, q2 = random_layer(oracle, rng, E, N, K)
    x = bf16(rng.standard_normal((T, K)))
    ids = rng.integers(-1, E + 1, size=(T, 8)).astype(np.int32)
    tw = rng.uniform(0, 1, size=(T, 8)).astype(np.float32)
    out, act = oracle.moe_w4a16(x, w13, q13, w2, q2, tw, ids, clamp_limit=10.0)

    def deq(words, sc):
        w = torch.from_numpy(words.astype(np.int64) & 0xFFFFFFFF)
        codes = torch.stack([(w >> (4 * i)) & 15 for i in range(8)], dim=-1).flatten(-2)
        s = torch.from_numpy(sc.astype(np.int32) << 16).view(torch.float32).double()
        return (codes.double() - 8) * s.repeat_interleave(32, dim=-1)

    to_bf = lambda v: v.float().to(torch.bfloat16).float()
    xt = torch.from_numpy(x.astype(np.int32) << 16).view(torch.float32).double()
    res = torch.zeros(T, K)
    for t in range(T):
        for j in range(8):
            e = int(ids[t, j])
            if not 0 <= e < E:
                continue
            c1 = to_bf(deq(w13[e], q13[e]) @ xt[t])
            g = c1[:N].clamp(max=10.0)
            u = c1[N:].clamp(-10.0, 10.0)
            c2 = to_bf(F.silu(g) * u)
            assert torch.equal(c2, torch.from_numpy(f32(act[8 * t + j])))
            y = (deq(w2[e], q2[e]) @ c2.double()).float()
            res[t] += to_bf(torch.tensor(float(tw[t, j])) * y)
    assert np.array_equal(f32(out), to_bf(res).numpy())
