"""GPU parity of the W4A16 group-32 MoE layer (repack, gate/up + SiLU with
clamp, down + router weights + route sum) against the oracle, at the GLM-5.3
TP4 decode shape: 288 experts, hidden 4096, intermediate 512, top-8, 1..8
tokens, the reference aligner's seven routing patterns
(benchmarks/moe_align.py:49-55).

Tolerances.  The kernels sum each 32-feature group on the matrix cores and
the groups in fp32 in another order than the oracle's exact dot, so a bf16
rounding point (c1, c2, c3) may land one ulp apart.  c2 (the activation) is
checked elementwise to |d| <= 2^-6 |ref| + 2^-10 (two bf16 ulps plus a
floor for values near zero); the layer output elementwise to
|d| <= 2^-7 |ref| + 2e-2 (one bf16 ulp of the value over the attention's
max-abs bar, which alone fits outputs of unit scale) and to mean-abs <=
2e-3 * max(1, mean |ref|).  The seeded random cases (any input scale and
clamp) are checked stage by stage instead (assert_stages_close): the
elementwise output bar above is a property of these inputs, not a bound.
The repack is integer work and is bit-exact."""
import random

import numpy as np
import pytest

import workloads as W
from conftest import log_case

pytestmark = pytest.mark.gpu

PATTERNS = ("distinct", "shared_top8", "random_top8", "all_one_expert", "seven_experts", "invalid_mixed",
            "all_invalid")


@pytest.fixture(scope="module")
def moe(cuda, oracle):
    import torch
    from titan_moe_w4a16 import repack_w4a16
    log_case("moe layer: build 288 x (1024 x 4096 + 4096 x 512) W4A16 weights")
    lay = W.moe_w4a16_layer(cuda, seed=W.SEED_FIXTURE)
    w13, s13 = repack_w4a16(lay["w13_packed"], lay["w13_scale"])
    w2, s2 = repack_w4a16(lay["w2_packed"], lay["w2_scale"])
    dev = {"w13": w13, "w2": w2, "w13_scale": s13, "w2_scale": s2}
    host = {k: v.cpu().numpy() if v.dtype != torch.bfloat16 else v.view(torch.int16).cpu().numpy().view(np.uint16)
            for k, v in lay.items()}
    torch.cuda.synchronize()
    return {"dev": dev, "host": host, "packed": lay, "cache": {}}


def run_oracle(oracle, moe, x, ids, tw, clamp=10.0):
    import torch
    h = moe["host"]
    xs = x.view(torch.int16).cpu().numpy().view(np.uint16)
    return oracle.moe_w4a16(xs, h["w13_packed"], h["w13_scale"], h["w2_packed"], h["w2_scale"],
                            tw.cpu().numpy(), ids.cpu().numpy(), clamp_limit=clamp, cache=moe["cache"])


def assert_out_close(got, want_u16, oracle, what):
    g = got.float().cpu().numpy()
    w = oracle.bf16_to_f32(want_u16)
    err = np.abs(g - w)
    excess = err - (2.0 ** -7 * np.abs(w) + 2e-2)
    mean_bar = 2e-3 * max(1.0, float(np.abs(w).mean()))
    assert excess.max() <= 0 and err.mean() <= mean_bar, \
        f"{what}: max {err.max():.3e} (excess {excess.max():.3e}) mean {err.mean():.3e} (bar {mean_bar:.2e})"
    return err


def assert_act_close(got, want_u16, rows, oracle, what):
    g = got.float().cpu().numpy()[rows]
    w = oracle.bf16_to_f32(want_u16)[rows]
    bad = np.abs(g - w) > 2.0 ** -6 * np.abs(w) + 2.0 ** -10
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} c2 values off, e.g. {g[bad][:4]} vs {w[bad][:4]}"


def bf16_ulp(v):
    return np.exp2(np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -126))) - 7)


def assert_stages_close(oracle, moe, x, out, act, want_out, ids, tw, clamp, what):
    """The layer checked stage by stage, a bar that holds for any inputs:
    c2 of every routed slot within the oracle's activation over the box of
    c1 values around the oracle's c1 -- one bf16 ulp (c1's fp32 order can
    flip its bf16 rounding; where SiLU is steep that moves c2 by several
    ulps) plus 2^-20 of the magnitude of c1's partial sums (16 fp32 ulps of
    them: a c1 near zero by cancellation carries that absolute error) --
    widened by one ulp of c2 for its own rounding; the output against the
    oracle's second half run on the kernel's own c2, where the only freedom
    left is the rounding of each slot's c3 = bf16(w * y) (y in fp32 order)
    -- one ulp of each |c3| -- and of the bf16 sum; and the mean error
    against the oracle's whole layer.  (A c3 flip moves an output by one ulp
    of that slot's c3, which can be far above the output itself when slots
    cancel, so a bar relative to |out| alone does not hold in general.)"""
    import torch
    h = moe["host"]
    ids_np = ids.cpu().numpy()
    routed = np.flatnonzero(((ids_np >= 0) & (ids_np < 288)).reshape(-1))
    xs = x.view(torch.int16).cpu().numpy().view(np.uint16)
    c1, mag = oracle.moe_w4a16_c1(xs, h["w13_packed"], h["w13_scale"], h["w2_packed"], h["w2_scale"], ids_np,
                                  moe["cache"], with_magnitude=True)
    c1, mag = c1[routed], mag[routed]
    n = c1.shape[1] // 2
    step = (bf16_ulp(c1) + 2.0 ** -20 * mag).astype(np.float32)
    corners = []
    for dg in (-1, 0, 1):
        for du in (-1, 0, 1):
            shift = np.concatenate([np.full(n, dg, np.float32), np.full(n, du, np.float32)])
            corners.append(oracle.moe_activation(c1 + shift * step, clamp))
    lo, hi = np.minimum.reduce(corners), np.maximum.reduce(corners)
    got_c2 = act.float().cpu().numpy()[routed]
    off = (got_c2 < lo - bf16_ulp(lo)) | (got_c2 > hi + bf16_ulp(hi))
    assert not off.any(), (f"{what}: {off.sum()} of {off.size} c2 values outside the one-ulp c1 box, "
                           f"e.g. {got_c2[off][:4]} in [{lo[off][:4]}, {hi[off][:4]}]")
    act_u16 = act.view(torch.int16).cpu().numpy().view(np.uint16)
    out_own, c3 = oracle.moe_w4a16_down(act_u16, h["w13_packed"], h["w13_scale"], h["w2_packed"], h["w2_scale"],
                                        tw.cpu().numpy(), ids_np, moe["cache"])
    g = out.float().cpu().numpy()
    w_own = oracle.bf16_to_f32(out_own)
    bound = bf16_ulp(c3).sum(axis=1) + bf16_ulp(w_own)
    over = np.abs(g - w_own) > bound
    assert not over.any(), (f"{what}: {over.sum()} outputs beyond the c3 rounding bound on the kernel's c2, "
                            f"e.g. {g[over][:4]} vs {w_own[over][:4]}")
    w = oracle.bf16_to_f32(want_out)
    mean_bar = 2e-3 * max(1.0, float(np.abs(w).mean()))
    assert np.abs(g - w).mean() <= mean_bar, f"{what}: mean {np.abs(g - w).mean():.3e} (bar {mean_bar:.2e})"


def test_repack_bit_exact(cuda, oracle, moe):
    import torch
    from titan_moe_w4a16 import repack_w4a16
    g = torch.Generator(device=cuda).manual_seed(5)
    small = torch.randint(0, 256, (3, 48, 192), generator=g, device=cuda, dtype=torch.uint8).view(torch.int32)
    small_s = torch.randint(0, 2**15, (3, 48, 12), generator=g, device=cuda, dtype=torch.int16).view(torch.bfloat16)
    log_case("repack [3, 48, 48] words")
    got, got_s = repack_w4a16(small, small_s)
    assert np.array_equal(got.cpu().numpy(), oracle.repack_w4a16(small.cpu().numpy()))
    assert np.array_equal(got_s.view(torch.int16).cpu().numpy(),
                          oracle.repack_w4a16_scales(small_s.view(torch.int16).cpu().numpy()))
    for name in ("w13", "w2"):
        want = oracle.repack_w4a16(moe["host"][name + "_packed"][[0, 141, 287]])
        assert np.array_equal(moe["dev"][name][[0, 141, 287]].cpu().numpy(), want), name
        want_s = oracle.repack_w4a16_scales(moe["host"][name + "_scale"][[0, 141, 287]])
        got_s = moe["dev"][name + "_scale"][[0, 141, 287]].view(torch.int16).cpu().numpy().view(np.uint16)
        assert np.array_equal(got_s, want_s), name + "_scale"


@pytest.mark.parametrize("batch", [1, 2, 4, 8])
@pytest.mark.parametrize("pattern", PATTERNS)
def test_fused_matches_oracle(cuda, oracle, moe, batch, pattern):
    import torch
    from titan_moe_w4a16 import fused_moe_w4a16
    flat = oracle.moe_patterns(batch, random.Random(37))[pattern]
    ids = torch.tensor(flat, dtype=torch.int32, device=cuda).view(batch, 8)
    g = torch.Generator(device=cuda).manual_seed(1000 * batch + PATTERNS.index(pattern))
    x, _, tw = W.moe_w4a16_inputs(batch, cuda, g, ids=ids)
    d = moe["dev"]
    log_case("fused moe", batch, pattern)
    out = fused_moe_w4a16(x, d["w13"], d["w2"], d["w13_scale"], d["w2_scale"], tw, ids)
    torch.cuda.synchronize()
    want, _ = run_oracle(oracle, moe, x, ids, tw)
    assert_out_close(out, want, oracle, f"B={batch} {pattern}")
    if pattern == "all_invalid":
        assert not out.float().abs().sum().item()


@pytest.mark.parametrize("batch", [1, 2, 4, 8])
def test_gate_up_activation_matches_oracle(cuda, oracle, moe, batch):
    """The first kernel alone, fed by the aligner: c2 of every routed slot."""
    import torch
    from titan_moe_align import titan_moe_align_small
    from titan_moe_w4a16 import moe_w4a16_gate_up, moe_w4a16_down, fused_moe_w4a16
    g = torch.Generator(device=cuda).manual_seed(77 + batch)
    x, ids, tw = W.moe_w4a16_inputs(batch, cuda, g)
    ids[0, :3] = ids[0, 4]                      # a shared expert: an aligner block with several slots
    d = moe["dev"]
    log_case("gate_up + down", batch)
    sorted_ids, expert_ids, _ = titan_moe_align_small(ids)
    act = moe_w4a16_gate_up(x, d["w13"], d["w13_scale"], sorted_ids, expert_ids)
    out = moe_w4a16_down(act, d["w2"], d["w2_scale"], tw, ids)
    torch.cuda.synchronize()
    want_out, want_act = run_oracle(oracle, moe, x, ids, tw)
    assert_act_close(act, want_act, np.arange(batch * 8), oracle, f"B={batch} c2")
    assert_out_close(out, want_out, oracle, f"B={batch} out")
    # the aligner kernel + two stages and the fused layer (alignment inside
    # its gate/up kernel) give the same bits
    fused = fused_moe_w4a16(x, d["w13"], d["w2"], d["w13_scale"], d["w2_scale"], tw, ids)
    torch.cuda.synchronize()
    assert torch.equal(out, fused), batch


def test_int64_ids_and_invalid_routes(cuda, oracle, moe):
    """int64 ids are compared at full width (5 + 2^32 is not expert 5) and
    every route outside [0, 288) contributes exactly nothing."""
    import torch
    from titan_moe_w4a16 import fused_moe_w4a16
    g = torch.Generator(device=cuda).manual_seed(91)
    x, ids, tw = W.moe_w4a16_inputs(4, cuda, g)
    ids64 = ids.to(torch.int64)
    ids64[0, 1] = 5 + 2 ** 32
    ids64[1, 0] = -1
    ids64[2, 7] = 288
    ids64[3, 3] = -(2 ** 40)
    d = moe["dev"]
    log_case("fused moe int64 ids with invalid routes")
    out = fused_moe_w4a16(x, d["w13"], d["w2"], d["w13_scale"], d["w2_scale"], tw, ids64)
    tw0 = tw.clone()
    for t, j in ((0, 1), (1, 0), (2, 7), (3, 3)):
        tw0[t, j] = 0
    ids_ok = torch.where((ids64 >= 0) & (ids64 < 288), ids64, torch.zeros_like(ids64)).to(torch.int32)
    ref = fused_moe_w4a16(x, d["w13"], d["w2"], d["w13_scale"], d["w2_scale"], tw0, ids_ok.contiguous())
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    want, _ = run_oracle(oracle, moe, x, ids64, tw)
    assert_out_close(out, want, oracle, "int64 invalid")


def test_clamp_off_row_stride_and_output(cuda, oracle, moe):
    import torch
    from titan_moe_w4a16 import fused_moe_w4a16
    g = torch.Generator(device=cuda).manual_seed(92)
    big = (3.0 * torch.randn(3, 4096 + 64, generator=g, device=cuda)).to(torch.bfloat16)
    x = big[:, 32:32 + 4096]                      # row stride 4160 elements, 64-byte aligned start
    _, ids, tw = W.moe_w4a16_inputs(3, cuda, g)
    d = moe["dev"]
    out = torch.full((3, 4096), 7.0, dtype=torch.bfloat16, device=cuda)
    log_case("fused moe, clamp off, strided rows, output=")
    ret = fused_moe_w4a16(x, d["w13"], d["w2"], d["w13_scale"], d["w2_scale"], tw, ids, clamp_limit=None,
                          output=out)
    assert ret.data_ptr() == out.data_ptr()
    clamped = fused_moe_w4a16(x, d["w13"], d["w2"], d["w13_scale"], d["w2_scale"], tw, ids)
    torch.cuda.synchronize()
    want, _ = run_oracle(oracle, moe, x, ids, tw, clamp=None)
    assert_out_close(out, want, oracle, "clamp off")
    want_c, _ = run_oracle(oracle, moe, x, ids, tw, clamp=10.0)
    assert_out_close(clamped, want_c, oracle, "clamp 10")
    assert not torch.equal(out, clamped)          # 3-sigma inputs push gate/up past 10


def test_random_routes_and_limits(cuda, oracle, moe):
    """Seeded random batch sizes, experts per slot (a token repeating an
    expert, ids outside [0, 288)), router weights, input scales and clamp
    limits: the fused layer equal to the aligner + two stages bit for bit,
    and checked stage by stage against the oracle (assert_stages_close)."""
    import torch
    from titan_moe_align import titan_moe_align_small
    from titan_moe_w4a16 import fused_moe_w4a16, moe_w4a16_down, moe_w4a16_gate_up
    rng = np.random.default_rng(9090)
    g = torch.Generator(device=cuda).manual_seed(9090)
    d = moe["dev"]
    for case in range(8):
        b = int(rng.integers(1, 9))
        ids = rng.integers(0, 288, size=(b, 8))
        if case % 3 == 1:
            ids[rng.random(ids.shape) < 0.2] = rng.choice([-1, 288, 1000])
        if case % 3 == 2:
            ids[0, 1] = ids[0, 0]                          # one token routes twice to an expert
        ids_t = torch.from_numpy(ids.astype(np.int32)).to(cuda)
        tw = torch.softmax(torch.randn(b, 8, generator=g, device=cuda), dim=1).contiguous()
        x = (torch.randn(b, 4096, generator=g, device=cuda) * float(rng.uniform(0.2, 3.0))).to(torch.bfloat16)
        clamp = float(rng.choice([10.0, 7.0, 25.0]))
        log_case("fused moe random", case, b, clamp)
        out = fused_moe_w4a16(x, d["w13"], d["w2"], d["w13_scale"], d["w2_scale"], tw, ids_t, clamp_limit=clamp)
        sorted_ids, expert_ids, _ = titan_moe_align_small(ids_t)
        act = moe_w4a16_gate_up(x, d["w13"], d["w13_scale"], sorted_ids, expert_ids, clamp_limit=clamp)
        staged = moe_w4a16_down(act, d["w2"], d["w2_scale"], tw, ids_t)
        torch.cuda.synchronize()
        assert torch.equal(out, staged), case          # the fused layer = aligner + the two stages
        want, _ = run_oracle(oracle, moe, x, ids_t, tw, clamp=clamp)
        assert_stages_close(oracle, moe, x, out, act, want, ids_t, tw, clamp, f"random case {case}")


def test_nan_token_propagates(cuda, oracle, moe):
    """A NaN in one token's hidden state makes that token's output NaN (the
    clamp keeps NaN, as torch.clamp does) and leaves the others exact."""
    import torch
    from titan_moe_w4a16 import fused_moe_w4a16
    g = torch.Generator(device=cuda).manual_seed(93)
    x, ids, tw = W.moe_w4a16_inputs(4, cuda, g)
    x[1, 100] = float("nan")
    d = moe["dev"]
    log_case("fused moe, NaN in token 1")
    out = fused_moe_w4a16(x, d["w13"], d["w2"], d["w13_scale"], d["w2_scale"], tw, ids)
    torch.cuda.synchronize()
    want, _ = run_oracle(oracle, moe, x, ids, tw)
    w = oracle.bf16_to_f32(want)
    o = out.float().cpu().numpy()
    assert np.isnan(w[1]).all() and np.isnan(o[1]).all()
    keep = [0, 2, 3]
    assert_out_close(out[keep], want[keep], oracle, "tokens without NaN")


@pytest.mark.parametrize("batch", [1, 8])
def test_graph_replay_deterministic(cuda, moe, batch):
    """Graph replays equal the eager call (B=1 takes the one-token gate/up
    path, B=8 the aligned blocks)."""
    import torch
    from titan_moe_w4a16 import fused_moe_w4a16
    g = torch.Generator(device=cuda).manual_seed(93)
    x, ids, tw = W.moe_w4a16_inputs(batch, cuda, g)
    d = moe["dev"]
    fn = lambda: fused_moe_w4a16(x, d["w13"], d["w2"], d["w13_scale"], d["w2_scale"], tw, ids)
    log_case("fused moe graph capture", batch)
    eager = fn()
    again = fn()
    torch.cuda.synchronize()
    assert torch.equal(eager, again)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = fn()
    for i in range(4):
        captured.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, eager), f"replay {i}"
        fn()                                          # eager work between replays
        torch.cuda.synchronize()


def test_whole_experts_n2048(cuda, oracle):
    """The gate's other width (profiles/sm74/titan_prefill/marlin.py:94:
    N = 2048, whole experts under pipeline parallelism): 288 x 4096 x 2048
    weights, two tokens, against the oracle on the experts the routes use."""
    import torch
    from titan_moe_w4a16 import fused_moe_w4a16, repack_w4a16
    log_case("moe layer N=2048: build 288 x (4096 x 4096 + 4096 x 2048) W4A16 weights")
    lay = W.moe_w4a16_layer(cuda, seed=W.SEED_FIXTURE + 7, inter=2048)
    w13, s13 = repack_w4a16(lay["w13_packed"], lay["w13_scale"])
    w2, s2 = repack_w4a16(lay["w2_packed"], lay["w2_scale"])
    g = torch.Generator(device=cuda).manual_seed(2048)
    x, ids, tw = W.moe_w4a16_inputs(2, cuda, g)
    ids[1, :2] = ids[0, :2]                       # two experts shared by both tokens
    log_case("fused moe N=2048 B=2")
    out = fused_moe_w4a16(x, w13, w2, s13, s2, tw, ids)
    torch.cuda.synchronize()
    used = torch.unique(ids.flatten().long())
    local = torch.searchsorted(used, ids.long()).to(torch.int32)
    pick = lambda t: t.index_select(0, used).contiguous()
    bits = lambda t: t.view(torch.int16).cpu().numpy().view(np.uint16)
    want, _ = oracle.moe_w4a16(bits(x), pick(lay["w13_packed"]).cpu().numpy(), bits(pick(lay["w13_scale"])),
                               pick(lay["w2_packed"]).cpu().numpy(), bits(pick(lay["w2_scale"])),
                               tw.cpu().numpy(), local.cpu().numpy())
    assert_out_close(out, want, oracle, "N=2048 B=2")


@pytest.mark.gpu
@pytest.mark.parametrize("hidden,inter", [(1024, 256), (640, 256), (1536, 128)])
def test_split_k_kernel_other_width(cuda, oracle, hidden, inter):
    """Hidden sizes other than 4096 take the split-K gate/up kernel (4096
    streams), at 1, 3 and 8 tokens (experts shared between tokens from B=3
    on), against the oracle on the experts the routes use.  640 (5 chunks of
    128 over 8 waves) and 1536 (12 chunks, 2 per wave) leave the last waves
    with no chunk: they must stage no activations (their offset lies past the
    row) and add nothing."""
    import torch
    from titan_moe_w4a16 import fused_moe_w4a16, repack_w4a16
    log_case(f"moe layer K={hidden} N={inter}: build 288 x ({2 * inter} x {hidden} + {hidden} x {inter}) weights")
    lay = W.moe_w4a16_layer(cuda, seed=W.SEED_FIXTURE + 11, hidden=hidden, inter=inter)
    w13, s13 = repack_w4a16(lay["w13_packed"], lay["w13_scale"])
    w2, s2 = repack_w4a16(lay["w2_packed"], lay["w2_scale"])
    g = torch.Generator(device=cuda).manual_seed(hidden)
    bits = lambda t: t.view(torch.int16).cpu().numpy().view(np.uint16)
    for batch in (1, 3, 8):
        x, ids, tw = W.moe_w4a16_inputs(batch, cuda, g, hidden=hidden)
        if batch > 1:
            ids[1, :3] = ids[0, :3]               # experts shared by two tokens: multi-slot blocks
        log_case(f"fused moe K={hidden} N={inter} B={batch}")
        out = fused_moe_w4a16(x, w13, w2, s13, s2, tw, ids)
        torch.cuda.synchronize()
        used = torch.unique(ids.flatten().long())
        local = torch.searchsorted(used, ids.long()).to(torch.int32)
        pick = lambda t: t.index_select(0, used).contiguous()
        want, _ = oracle.moe_w4a16(bits(x), pick(lay["w13_packed"]).cpu().numpy(), bits(pick(lay["w13_scale"])),
                                   pick(lay["w2_packed"]).cpu().numpy(), bits(pick(lay["w2_scale"])),
                                   tw.cpu().numpy(), local.cpu().numpy())
        assert_out_close(out, want, oracle, f"K={hidden} N={inter} B={batch}")
