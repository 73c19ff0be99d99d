#!/usr/bin/env python3
"""Benchmark of the GLM-5.3 decode hot path on one MI355X.

Headline: sparse NoPE MLA decode at B=8 over a 262144-row INT8 cache with
2176 indices per query (16 heads, one KV head).  A step is one call of
triton_mla_sparse_attention; it is captured once in a HIP graph and replayed
(the reference's protocol, benchmarks/mla.py:38-55): W untimed replays, then K
timed replays bracketed by device synchronisation, timed with events on the
stream the kernels run on; by default up to 20 steps (the largest divisor of
K up to 20) are captured back to back in one graph, as decode steps sit inside
one captured model step in serving (each graph boundary adds about 4 us to
the step after it; --unroll 1 gives the reference's one-call-per-replay
figure, also reported).  `value` is achieved algorithmic GB/s of the step
(gathered valid 528-byte rows + indices + q + out) with inputs resident in
HBM: consecutive steps read 256 different caches, more rows between two
visits of one cache than the 256 MB Infinity Cache holds; warm = one cache
replayed (its rows stay in the Infinity Cache, as in the reference's
measurements); the cold figures flush it (a 1 GiB write) before every timed
step.

Extra fields: the B=1 decode, the 262144-row store_int8 writer, the MoE
align (16 calls per graph, as docs/measurements.json:1445 records), the W4A16
MoE layer (B=1..8), the sparse indexer's decode scoring (FP8 paged logits
and top-512 pools over 65536 pools per request, B=1 and B=8), the
prefill-shaped T=2048 call, and the CPU baseline (the C oracle on the host
cores, a bounded sample of the same workload).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]
Prints one JSON line on stdout.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (str(ROOT), str(ROOT / "glm-5.3-kernels_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBS = 8000.0
FP8_PEAK_FLOPS = 5.0e15   # MI355X dense FP8 matrix peak
METRIC = "sparse-MLA decode µs/step + achieved HBM GB/s, B1/B8, 262k ctx, 2176 idx"


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


class Timer:
    """Events recorded on the current stream (the one the kernels use).

    One untimed replay of the same graph runs just before a timed region
    (no synchronisation between them), so the GPU is busy while the host
    queues the timed replays: the region then times k replays that follow
    each other as the steps of a decode loop do, rather than also the
    graph launch latency of its first replay, which a short run (k = 2
    replays of a 10-step graph) would spread over its few steps (B=8 over
    the rotation: 11.97 -> 11.90 us per step at k = 2, 11.72 at k = 20
    either way)."""

    def __init__(self, torch):
        self.torch = torch

    def replay_loop(self, graph, k: int) -> float:
        torch = self.torch
        torch.cuda.synchronize()
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        graph.replay()   # untimed lead replay
        s.record()
        for _ in range(k):
            graph.replay()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) * 1e3 / k          # us per replay

    def warm_clocks(self, graph, min_ms: float = 20.0) -> None:
        """Untimed replays for at least min_ms of GPU time: out of idle the
        part runs its first milliseconds at lower clocks (B=8 over the
        rotation, 2-replay samples: 12.17 us per step right after 0.5 s idle,
        11.92 after 200 replays), and a decode loop runs at busy clocks."""
        torch = self.torch
        torch.cuda.synchronize()
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record()
        done = 0.0
        while done < min_ms:
            for _ in range(10):
                graph.replay()
            e.record()
            torch.cuda.synchronize()
            done = s.elapsed_time(e)

    def median_loop(self, graph, k: int, samples: int = 5) -> float:
        """Median over `samples` timings of k replays (us per replay), after
        warm_clocks."""
        self.warm_clocks(graph)
        return statistics.median(self.replay_loop(graph, k) for _ in range(samples))

    def cold_loop(self, graph, k: int, flush) -> float:
        torch = self.torch
        evs = []
        for _ in range(k):
            flush()
            s = torch.cuda.Event(enable_timing=True)
            e = torch.cuda.Event(enable_timing=True)
            s.record()
            graph.replay()
            e.record()
            evs.append((s, e))
        torch.cuda.synchronize()
        return statistics.median(s.elapsed_time(e) * 1e3 for s, e in evs)


def cpu_model() -> str:
    """The host CPU's model name (as lscpu prints it), from /proc/cpuinfo."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_time(fn, min_s: float, per_call: int = 1) -> float:
    """The CPU baseline's timing: 3 warm-up calls of fn, then 5 samples, each
    repeating fn until at least min_s seconds have passed; the median of the
    samples' mean time per call, in us (fn runs per_call calls each)."""
    for _ in range(3):
        fn()
    samples = []
    for _ in range(5):
        n = 0
        t0 = time.perf_counter()
        while True:
            fn()
            n += 1
            el = time.perf_counter() - t0
            if el >= min_s:
                break
        samples.append(el / (n * per_call) * 1e6)
    return statistics.median(samples)


def split_kernel_threads(topk: int, splits: int) -> int:
    """Threads per workgroup of the decode split kernel the library launches
    for this split length: 12 waves (three key groups) for splits of 65-96
    keys, 8 waves otherwise (splits past 256 keys take the 2-wave pair
    kernel, which the decode workloads never reach)."""
    split_len = -(-topk // splits)
    return 768 if 64 < split_len <= 96 else 512


def capture(torch, fn, unroll: int = 1):
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(unroll):
            out = fn()
    torch.cuda.synchronize()
    return g, out


# Decode steps over HBM-resident caches: consecutive steps read different
# layers' caches, as a model's layers do.  A step touches only its own rows
# (8.8 MB at B=8, 1.1 MB at B=1), so the rotation needs enough caches that the
# rows touched between two visits of one cache exceed the 256 MB MALL: 256
# caches of 262144 rows (35 GB of HBM).  With 5 caches (46 MB touched per
# cycle at B=8) the B=8 step read 11.12 us per step against 11.35 us over 64
# or 256 caches, its split kernel 7.31 against 7.55 us.
ROT_CACHES = 256
# W4A16 MoE layer over HBM: calls with fresh routes cycle over 4 layers' expert
# weights (1.02 GB each); 32 calls per graph read at least 32 x 28 MB (B=1,
# 8 experts of 3.5 MB) between two visits of one call's experts, more than the
# MALL holds.
MOE_ROT_CALLS = 32


def rotation_caches(torch, W, store_int8, first, n: int, n_rows: int) -> list:
    """`first` and n - 1 more 262144-row caches: up to four with contents of
    their own (latents stored by store_int8), the others copies of those at
    their own addresses (the timing reads rows, the values do not matter)."""
    caches = [first]
    for li in range(1, min(n, 5)):
        _, xr, cr, sr = W.decode_cache(first.device, seed=W.SEED_BENCH + 300 + li, dist="t3")
        store_int8(xr, cr, sr)
        del xr
        caches.append(cr.view(n_rows, 1, W.ROW_BYTES))
    base = len(caches)
    for i in range(base, n):
        caches.append(caches[i % base].clone())
    torch.cuda.synchronize()
    return caches


class Cycle:
    """Graphs replayed in turn: each replay() runs the next one.  Graph j of
    a rotation runs steps unroll*j .. unroll*(j+1) - 1, each step on its own
    cache, so k replays time exactly k * unroll steps while the steps keep
    cycling over every cache of the rotation."""

    def __init__(self, graphs):
        self.graphs, self.i = graphs, 0

    def replay(self):
        self.graphs[self.i].replay()
        self.i = (self.i + 1) % len(self.graphs)


def rotation_cycle(torch, caches, fn, unroll: int) -> Cycle:
    """A Cycle of ceil(len(caches) / unroll) graphs of `unroll` calls
    fn(cache), call i of the cycle on cache i % len(caches)."""
    n = len(caches)
    graphs = []
    for j in range(-(-n // unroll)):
        g, _ = capture(torch, lambda j=j: [fn(caches[(unroll * j + i) % n]) for i in range(unroll)], 1)
        graphs.append(g)
    return Cycle(graphs)


def stream_ceilings(torch, timer, dev, nbytes: int = 1 << 30) -> dict:
    """The part's streaming rates through glm53_stream_probe (GB/s): 16-byte
    lane reads of nbytes with plain and with non-temporal loads, and a
    non-temporal copy of nbytes (read + write bytes counted), each 3 calls
    per graph, median of 5 samples -- the ceilings the bandwidth-bound
    kernels are read against."""
    import _glm53_lib as lib
    L = lib.load()
    src = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(7)
    dst = torch.empty_like(src)
    out = {}
    for kind, name, moved in ((0, "read", nbytes), (1, "read_nt", nbytes), (2, "copy_nt", 2 * nbytes)):
        def call(kind=kind):   # the current stream: under graph capture, the capturing one
            lib.check(L.glm53_stream_probe(kind, src.data_ptr(), dst.data_ptr(), nbytes, lib.stream_handle(dev)),
                      "glm53_stream_probe")
        g, _ = capture(torch, call, 3)
        g.replay()
        us = timer.median_loop(g, 5) / 3
        out[f"{name}_gbs"] = round(moved / (us * 1e-6) / 1e9, 1)
        del g
    del src, dst
    return out


def run_case(args, torch, W, dev, timer, g8, kv8, cache8, q8, idx8, n_rows, cu):
    """One workload alone, for kernel profiles (rocprofv3 --kernel-trace /
    --pmc over exactly these dispatches)."""
    from titan_kv import store_int8
    from titan_mla import triton_mla_sparse_attention, sparse_mla_partials, _choose_num_kv_splits_mi355x
    K, unroll = args.steps, args.unroll
    if args.case == "moe_align":
        # the reference's protocol: 16 calls per graph, median of 5 samples of 100 replays
        from titan_moe_align import titan_moe_align_small
        ids = W.moe_routes(args.batch, dev, W.gen(dev, W.SEED_BENCH))
        mg, _ = capture(torch, lambda: titan_moe_align_small(ids), unroll=16)
        for _ in range(5):
            mg.replay()
        us = statistics.median(timer.replay_loop(mg, 100) / 16 for _ in range(5))
        log(f"case moe_align B={args.batch}: {us:.3f} us per call (16 per graph, median of 5 x 100 replays)")
        return
    if args.case == "moe_layer":
        # the fused W4A16 MoE layer at --batch tokens, MOE_ROT_CALLS calls per
        # graph (fresh routes each) over 4 layers' expert weights
        from titan_moe_w4a16 import fused_moe_w4a16, repack_w4a16
        layers = []
        for li in range(4):
            lay = W.moe_w4a16_layer(dev, seed=W.SEED_BENCH + 100 + li)
            layers.append(repack_w4a16(lay["w13_packed"], lay["w13_scale"]) +
                          repack_w4a16(lay["w2_packed"], lay["w2_scale"]))
            del lay
        gmw = W.gen(dev, W.SEED_BENCH + args.batch)
        calls = []
        for i in range(MOE_ROT_CALLS):
            xm, idm, twm = W.moe_w4a16_inputs(args.batch, dev, gmw)
            calls.append((xm, idm, twm, layers[i % 4]))
        mg, _ = capture(torch, lambda: [fused_moe_w4a16(c[0], c[3][0], c[3][2], c[3][1], c[3][3], c[2], c[1])
                                        for c in calls], 1)
        for _ in range(3):
            mg.replay()
        us = timer.median_loop(mg, max(1, K // len(calls))) / len(calls)
        mb = statistics.mean(W.moe_w4a16_bytes(c[1], args.batch) for c in calls)
        log(f"case moe_layer B={args.batch}: {us:.3f} us per call, {mb / (us * 1e-6) / 1e9:.1f} GB/s algorithmic "
            f"({mb:.0f} B mean), {len(calls)} calls per graph over 4 layers")
        return
    if args.case == "dispatch_floor":
        # a kernel that adds 1 to one int32, 16 per graph: the MoE align protocol's floor
        one = torch.zeros(1, dtype=torch.int32, device=dev)
        fg, _ = capture(torch, lambda: one.add_(1), unroll=16)
        for _ in range(5):
            fg.replay()
        us = statistics.median(timer.replay_loop(fg, 100) / 16 for _ in range(5))
        log(f"case dispatch_floor: {us:.3f} us per kernel (16 per graph, median of 5 x 100 replays)")
        return
    if args.case == "stream":
        c = stream_ceilings(torch, timer, dev)
        log(f"case stream: 1 GiB read {c['read_gbs']} GB/s, non-temporal read {c['read_nt_gbs']} GB/s, "
            f"non-temporal copy {c['copy_nt_gbs']} GB/s (read + write)")
        return
    if args.case == "copy":
        # the same box's device copy: the practical HBM ceiling (read + write bytes)
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(3)
        dst = torch.empty_like(src)
        cg, _ = capture(torch, lambda: dst.copy_(src), unroll=3)
        cg.replay()
        us = timer.median_loop(cg, 5) / 3
        log(f"case copy: 1 GiB device copy {us:.1f} us, {2 * (1 << 30) / (us * 1e-6) / 1e9:.1f} GB/s (read + write)")
        return
    first = kv8
    if args.case in ("decode_b1", "decode_b1_split"):
        g1, x1, cache1, slots1 = W.decode_cache(dev, seed=W.SEED_BENCH + 1, dist="normal")
        store_int8(x1, cache1, slots1)
        del x1
        q1, idx1 = W.decode_b1_inputs(dev, g1)
        first = cache1.view(n_rows, 1, W.ROW_BYTES)
    caches = [first]
    if args.case != "writer_rotation":
        caches = rotation_caches(torch, W, store_int8, first, max(1, args.rotate), n_rows)
    turn = [0]

    def next_cache():
        turn[0] += 1
        return caches[(turn[0] - 1) % len(caches)]
    if args.case == "writer_scattered":
        # the prefill-shaped call's write: 2048 rows -> randperm slots of a 262144-row cache
        _, _, new_rows, slots = W.prefill_inputs(dev, g8)
        fn = lambda: store_int8(new_rows, cache8, slots)
        nbytes = W.writer_bytes(new_rows.shape[0])
    elif args.case == "prefill":
        qp, idxp, _, _ = W.prefill_inputs(dev, g8)
        fn = lambda: triton_mla_sparse_attention(qp, next_cache(), idxp, W.SM_SCALE, num_kv_splits=args.splits)
        nbytes = W.mla_bytes(idxp, n_rows)
    elif args.case == "decode_b1":
        # the B=1 step (split + merge)
        fn = lambda: triton_mla_sparse_attention(q1, next_cache(), idx1, W.SM_SCALE, num_kv_splits=args.splits)
        nbytes = W.mla_bytes(idx1, n_rows)
    elif args.case == "decode_b1_split":
        # the B=1 split kernel alone at the auto split count
        s1 = args.splits or _choose_num_kv_splits_mi355x(1, 1, W.TOPK, cu)
        fn = lambda: sparse_mla_partials(q1, next_cache(), idx1, W.SM_SCALE, s1)
        nbytes = W.mla_bytes(idx1, n_rows)
    elif args.case == "decode_b8":
        # the B=8 step (split + merge), the headline's call
        fn = lambda: triton_mla_sparse_attention(q8, next_cache(), idx8, W.SM_SCALE, num_kv_splits=args.splits)
        nbytes = W.mla_bytes(idx8, n_rows)
    elif args.case == "writer_rotation":
        # store_int8 of 262144 N(0,1) rows, cycling over `rotate` latent/cache sets
        sets = []
        for li in range(max(1, args.rotate)):
            _, xw, cw, sw = W.decode_cache(dev, seed=W.SEED_BENCH + 500 + li, dist="normal")
            sets.append((xw, cw, sw))
        turn_w = [0]

        def fn():
            turn_w[0] += 1
            xw, cw, sw = sets[(turn_w[0] - 1) % len(sets)]
            return store_int8(xw, cw, sw)
        caches = sets
        nbytes = W.writer_bytes(n_rows)
    elif args.case == "indexer_prefill":
        # 2048 query rows at the end of a 262144-token context: logits over
        # 65536 pools, then the top 512 per row
        from sparse_indexer import fp8_paged_mqa_logits, indexer_topk
        gi = W.gen(dev, W.SEED_BENCH + 2048)
        qpi, cpi, wpi, lpi, bpi, npi = W.indexer_prefill_inputs(dev, gi)
        fn = lambda: indexer_topk(fp8_paged_mqa_logits(qpi, cpi, wpi, lpi, bpi, npi, clean_logits=False), lpi,
                                  W.INDEX_TOPK_POOLS)
        # rows share their keys: the logits' bound is the matrix cores, so
        # report FLOP/s (the GB/s below counts each row's keys once per row)
        log(f"case indexer_prefill: logits {W.indexer_flops(lpi) / 1e12:.3f} TFLOP per call")
        nbytes = W.indexer_bytes(lpi)
    else:   # decode_b8_split: the split kernel alone at the auto split count
        s8 = args.splits or _choose_num_kv_splits_mi355x(8, 1, W.TOPK, cu)
        fn = lambda: sparse_mla_partials(q8, next_cache(), idx8, W.SM_SCALE, s8)
        nbytes = W.mla_bytes(idx8, n_rows)
    # graphs of `unroll` calls replayed in turn (the main run's rotation
    # protocol), each call reading the next cache of the rotation
    fn()
    torch.cuda.synchronize()
    graphs = []
    for _ in range(-(-len(caches) // unroll)):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(unroll):
                fn()
        graphs.append(g)
    torch.cuda.synchronize()
    gr = Cycle(graphs)
    for _ in range(max(1, args.warmup // unroll)):
        gr.replay()
    us = timer.median_loop(gr, max(1, K // unroll)) / unroll
    log(f"case {args.case}: {us:.3f} us per call, {nbytes / (us * 1e-6) / 1e9:.1f} GB/s algorithmic "
        f"({nbytes} B), {K} calls, {unroll} per graph, {len(graphs)} graph(s), {len(caches)} cache(s)")


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--quick", action="store_true", help="headline only: skip extras and CPU baseline")
    ap.add_argument("--rotate", type=int, default=1,
                    help="with --case: cycle the calls over this many 262144-row caches (or writer sets); "
                         "decode steps read their rows from HBM with the main run's 256")
    ap.add_argument("--case", choices=("writer_scattered", "writer_rotation", "prefill", "decode_b1",
                                       "decode_b1_split", "decode_b8", "decode_b8_split", "indexer_prefill",
                                       "moe_align", "moe_layer", "dispatch_floor", "copy", "stream"),
                    default=None,
                    help="time one workload alone (K calls, one per graph replay unless --unroll), print "
                         "its figure to stderr and exit: the command behind a kernel profile")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--batch", type=int, default=8, choices=(1, 2, 4, 8),
                    help="tokens for --case moe_align / moe_layer")
    ap.add_argument("--cpu-sample-s", type=float, default=1.0,
                    help="minimum length of one CPU-baseline timing sample (seconds)")
    ap.add_argument("--splits", type=int, default=None, help="force num_kv_splits for the decode calls")
    ap.add_argument("--sweep", action="store_true",
                    help="print a decode latency table over split counts (stderr) and exit")
    ap.add_argument("--unroll", type=int, default=None,
                    help="decode steps captured back to back per graph (K must be a multiple; default: the "
                         "largest divisor of K up to 20)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a 256 MiB device copy (the HBM byte-counter calibration) and exit")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the library runs the hot path at the per-rank shape on a "
              "single MI355X; multi-GPU runs are not part of it.", file=sys.stderr)
        sys.exit(2)
    if args.unroll is None and args.steps >= 1:
        args.unroll = max(d for d in range(1, 21) if args.steps % d == 0)
    if args.steps < 1 or args.warmup < 0 or args.unroll < 1 or args.steps % args.unroll:
        ap.error("steps >= 1, warmup >= 0, steps a multiple of unroll")

    import numpy as np
    import torch

    import workloads as W
    from titan_kv import store_int8
    from titan_mla import triton_mla_sparse_attention, _choose_num_kv_splits_mi355x
    from titan_moe_align import titan_moe_align_small

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    props = torch.cuda.get_device_properties(dev)
    cu = props.multi_processor_count
    timer = Timer(torch)
    flush_buf = torch.empty(1 << 30, dtype=torch.uint8, device=dev)

    def flush():
        flush_buf.fill_(1)

    K, Wm = args.steps, args.warmup
    extra = {}

    if args.copy_calibration:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(3)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("copy calibration: 5 copies of 268435456 bytes")
        return

    # ---------------------------------------------------------------- caches
    log("building 262144-row caches")
    g8, x8, cache8, slots8 = W.decode_cache(dev, seed=W.SEED_BENCH, dist="t3")
    store_int8(x8, cache8, slots8)
    n_rows = cache8.shape[0] * W.BLOCK
    kv8 = cache8.view(n_rows, 1, W.ROW_BYTES)
    q8, idx8 = W.decode_b8_inputs(dev, g8)
    del x8

    if args.case:
        run_case(args, torch, W, dev, timer, g8, kv8, cache8, q8, idx8, n_rows, cu)
        return

    if args.sweep:
        g1s, x1s, cache1s, slots1s = W.decode_cache(dev, seed=W.SEED_BENCH + 1, dist="normal")
        store_int8(x1s, cache1s, slots1s)
        del x1s
        q1s, idx1s = W.decode_b1_inputs(dev, g1s)
        kv1s = cache1s.view(n_rows, 1, W.ROW_BYTES)
        for name, q_, kv_, idx_ in (("b1", q1s, kv1s, idx1s), ("b8", q8, kv8, idx8)):
            for sp in (1, 2, 4, 8, 16, 17, 32, 34, 64, 68):
                for unroll in (1, 10):
                    gr, _ = capture(torch, lambda: triton_mla_sparse_attention(q_, kv_, idx_, W.SM_SCALE,
                                                                               num_kv_splits=sp), unroll)
                    for _ in range(10):
                        gr.replay()
                    us = timer.replay_loop(gr, 50) / unroll
                    usc = timer.cold_loop(gr, 20, flush) / unroll
                    log(f"sweep {name} splits={sp:3d} unroll={unroll:2d} warm {us:8.2f} us  cold {usc:8.2f} us")
                    del gr
        return

    # ---------------------------------------------------------------- headline: B=8
    # HBM-resident (the headline): consecutive steps read different layers'
    # caches (ROT_CACHES of them, same q and indices per step), `unroll`
    # steps per captured graph.  Warm (one cache replayed, MALL-resident, the
    # reference's protocol) is reported beside it.
    log(f"building the {ROT_CACHES}-cache layer rotation")
    rot = rotation_caches(torch, W, store_int8, kv8, ROT_CACHES, n_rows)

    def rotation(fn):
        """Steps fn(cache) over the rotation, `unroll` per graph."""
        return rotation_cycle(torch, rot, fn, args.unroll)

    def mla_b8(kv=kv8):
        return triton_mla_sparse_attention(q8, kv, idx8, W.SM_SCALE, num_kv_splits=args.splits)

    from titan_mla import sparse_mla_partials
    s8 = args.splits or _choose_num_kv_splits_mi355x(8, 1, W.TOPK, cu)
    bytes8 = W.mla_bytes(idx8, n_rows)
    n_samples = 5
    graph8r = rotation(mla_b8)
    for _ in range(max(1, Wm // args.unroll)):
        graph8r.replay()
    log(f"decode_b8: timing {n_samples} samples of {K} steps (splits={s8}, {args.unroll} per graph, "
        f"cycling {len(rot)} caches)")
    us8 = timer.median_loop(graph8r, K // args.unroll, n_samples) / args.unroll
    gbs8 = bytes8 / (us8 * 1e-6) / 1e9
    # the dominant kernel alone (first stage: split attention -> partials), same rotation
    pgr = rotation(lambda kv: sparse_mla_partials(q8, kv, idx8, W.SM_SCALE, s8))
    for _ in range(max(1, Wm // args.unroll)):
        pgr.replay()
    us8_kernel = timer.median_loop(pgr, K // args.unroll, n_samples) / args.unroll
    del graph8r, pgr
    # warm: one cache replayed (MALL-resident)
    graph8, _ = capture(torch, mla_b8, args.unroll)
    for _ in range(Wm):
        graph8.replay()
    us8_warm = timer.median_loop(graph8, K // args.unroll, n_samples) / args.unroll
    del graph8
    pg, _ = capture(torch, lambda: sparse_mla_partials(q8, kv8, idx8, W.SM_SCALE, s8), args.unroll)
    for _ in range(Wm):
        pg.replay()
    us8_kernel_warm = timer.median_loop(pg, K // args.unroll, n_samples) / args.unroll
    del pg
    # the floor under the step: the split kernel's memory chain alone (same
    # grid, index loads, row gathers, partial stores; no arithmetic) + the merge
    from titan_mla import sparse_mla_gather_floor, sparse_mla_merge
    floor_step = lambda kv: sparse_mla_merge(sparse_mla_gather_floor(q8, kv, idx8, s8), 8, 16, s8)
    fgr = rotation(floor_step)
    fgk = rotation(lambda kv: sparse_mla_gather_floor(q8, kv, idx8, s8))
    for _ in range(max(1, Wm // args.unroll)):
        fgr.replay()
        fgk.replay()
    us8_floor_step = timer.median_loop(fgr, K // args.unroll, n_samples) / args.unroll
    us8_floor_kernel = timer.median_loop(fgk, K // args.unroll, n_samples) / args.unroll
    del fgr, fgk
    g8_1, _ = capture(torch, mla_b8, 1)
    us8_cold = timer.cold_loop(g8_1, min(K, 50), flush)
    us8_single = timer.median_loop(g8_1, min(K, 100), n_samples)
    del g8_1
    extra["decode_b8"] = {"us_per_step_layer_rotation": round(us8, 3), "us_per_step_warm": round(us8_warm, 3),
                          "us_per_step_cold": round(us8_cold, 3),
                          "us_per_step_one_call_per_graph": round(us8_single, 3),
                          "us_split_kernel_alone_layer_rotation": round(us8_kernel, 3),
                          "us_split_kernel_alone_warm": round(us8_kernel_warm, 3),
                          "us_floor_step_layer_rotation": round(us8_floor_step, 3),
                          "us_floor_split_kernel_layer_rotation": round(us8_floor_kernel, 3),
                          "algorithmic_bytes": bytes8, "gbs_layer_rotation": round(gbs8, 1),
                          "gbs_warm": round(bytes8 / (us8_warm * 1e-6) / 1e9, 1),
                          "gbs_cold": round(bytes8 / (us8_cold * 1e-6) / 1e9, 1), "num_kv_splits": s8,
                          "flops": W.mla_flops(idx8, n_rows)}

    cpu = None
    if not args.quick:
        # ------------------------------------------------------------ B=1
        g1, x1, cache1, slots1 = W.decode_cache(dev, seed=W.SEED_BENCH + 1, dist="normal")
        torch.cuda.synchronize()
        # writer: 262144 rows, N(0,1) (the full-context writer configuration)
        wg, _ = capture(torch, lambda: store_int8(x1, cache1, slots1))
        for _ in range(max(1, Wm // 4)):
            wg.replay()
        log("store_int8 262144 rows")
        us_w = timer.replay_loop(wg, max(5, K // 10))
        us_w_cold = timer.cold_loop(wg, 10, flush)
        wb = W.writer_bytes(x1.shape[0])
        del wg
        # HBM-resident: three calls per graph cycling over three latent/cache
        # sets (3 x 406 MB, more than the 256 MB MALL), no flush inside the
        # sample; beside it the same box's device copy (1 GiB -> 1 GiB, read +
        # write bytes) as the practical ceiling of a streaming kernel.
        wsets = [(x1, cache1, slots1)]
        for li in range(2):
            _, xw, cw, sw = W.decode_cache(dev, seed=W.SEED_BENCH + 500 + li, dist="normal")
            wsets.append((xw, cw, sw))
        wgr, _ = capture(torch, lambda: [store_int8(xw, cw, sw) for xw, cw, sw in wsets])
        wgr.replay()
        us_w_rot = timer.median_loop(wgr, max(2, K // 10)) / len(wsets)
        del wgr, wsets
        csrc = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(3)
        cdst = torch.empty_like(csrc)
        cgr, _ = capture(torch, lambda: cdst.copy_(csrc), unroll=3)
        cgr.replay()
        us_copy = timer.median_loop(cgr, 5) / 3
        copy_gbs = 2 * (1 << 30) / (us_copy * 1e-6) / 1e9
        del cgr, csrc, cdst
        extra["hbm_stream_ceilings"] = dict(stream_ceilings(torch, timer, dev), device_copy_gbs=round(copy_gbs, 1),
                                            what="glm53_stream_probe over 1 GiB: plain and non-temporal 16-byte "
                                                 "lane reads, non-temporal copy (read + write bytes); "
                                                 "torch's device copy beside")
        gbs_w_rot = wb / (us_w_rot * 1e-6) / 1e9
        extra["store_int8_262144"] = {"us_per_call_hbm_rotation": round(us_w_rot, 2),
                                      "us_per_call_warm": round(us_w, 2), "us_per_call_cold": round(us_w_cold, 2),
                                      "algorithmic_bytes": wb, "gbs_hbm_rotation": round(gbs_w_rot, 1),
                                      "hbm_frac_rotation": round(gbs_w_rot / HBM_PEAK_GBS, 3),
                                      "device_copy_gbs": round(copy_gbs, 1),
                                      "frac_of_device_copy": round(gbs_w_rot / copy_gbs, 3),
                                      "gbs_warm": round(wb / (us_w * 1e-6) / 1e9, 1),
                                      "gbs_cold": round(wb / (us_w_cold * 1e-6) / 1e9, 1),
                                      "hbm_frac_cold": round(wb / (us_w_cold * 1e-6) / 1e9 / HBM_PEAK_GBS, 3),
                                      "rotation": "3 calls per graph over 3 sets of 262144 N(0,1) rows "
                                                  "(latents 268 MB + cache 138 MB each), median of 5 samples",
                                      "device_copy": "torch copy_ of 1 GiB into 1 GiB, 3 per graph, "
                                                     "(read + write bytes) / time",
                                      "cold": "1 GiB device write before each call (may leave dirty lines "
                                              "written back inside the timed call)"}
        kv1 = cache1.view(n_rows, 1, W.ROW_BYTES)
        q1, idx1 = W.decode_b1_inputs(dev, g1)
        del x1
        s1 = args.splits or _choose_num_kv_splits_mi355x(1, 1, W.TOPK, cu)
        mla_b1 = lambda: triton_mla_sparse_attention(q1, kv1, idx1, W.SM_SCALE, num_kv_splits=args.splits)
        graph1, _ = capture(torch, mla_b1, args.unroll)
        for _ in range(Wm):
            graph1.replay()
        log("decode_b1")
        us1 = timer.median_loop(graph1, K // args.unroll) / args.unroll
        g1_1, _ = capture(torch, mla_b1, 1)
        us1_cold = timer.cold_loop(g1_1, min(K, 50), flush)
        us1_single = timer.median_loop(g1_1, min(K, 100))
        del g1_1
        bytes1 = W.mla_bytes(idx1, n_rows)
        extra["decode_b1"] = {"us_per_step_warm": round(us1, 3), "us_per_step_cold": round(us1_cold, 3),
                              "us_per_step_one_call_per_graph": round(us1_single, 3),
                              "algorithmic_bytes": bytes1, "gbs_warm": round(bytes1 / (us1 * 1e-6) / 1e9, 1),
                              "gbs_cold": round(bytes1 / (us1_cold * 1e-6) / 1e9, 1), "num_kv_splits": s1}
        del graph1

        # ------------------------------------------------------------ the whole path, B=8
        # One decode step of the path in one graph: the 8 new tokens' rows
        # written into the cache (scattered slots), the sparse MLA decode over
        # it, and the MoE align of the 8 tokens' routes (launch gaps included).
        gp = W.gen(dev, W.SEED_BENCH + 400)
        x_new = torch.randn(8, 512, generator=gp, device=dev).to(torch.bfloat16)
        slots_new = torch.randperm(n_rows, generator=gp, device=dev)[:8]
        ids_new = W.moe_routes(8, dev, gp)

        def path_step():
            store_int8(x_new, cache8, slots_new)
            out = triton_mla_sparse_attention(q8, kv8, idx8, W.SM_SCALE, num_kv_splits=args.splits)
            titan_moe_align_small(ids_new)
            return out
        gps, _ = capture(torch, path_step, args.unroll)
        for _ in range(3):
            gps.replay()
        log("decode path B=8 (write + attention + align)")
        extra["decode_path_b8_us_per_step"] = round(timer.replay_loop(gps, max(2, K // args.unroll // 2))
                                                    / args.unroll, 3)
        del gps

        # ------------------------------------------------------------ B=1 layer rotation
        # B=1 over its own cache and the other rotation caches (HBM-resident).
        rot1 = [kv1] + rot[1:]
        grr = rotation_cycle(torch, rot1, lambda kv: triton_mla_sparse_attention(q1, kv, idx1, W.SM_SCALE,
                                                                                 num_kv_splits=args.splits),
                             args.unroll)
        for _ in range(3):
            grr.replay()
        log("decode_b1 layer rotation")
        us_r = timer.median_loop(grr, max(1, K // args.unroll)) / args.unroll
        extra["decode_b1"]["us_per_step_layer_rotation"] = round(us_r, 3)
        extra["decode_b1"]["gbs_layer_rotation"] = round(bytes1 / (us_r * 1e-6) / 1e9, 1)
        # B=1's floor: its split kernel's memory chain + the merge, same rotation
        from titan_mla import sparse_mla_gather_floor, sparse_mla_merge
        fg1 = rotation_cycle(torch, rot1, lambda kv: sparse_mla_merge(sparse_mla_gather_floor(q1, kv, idx1, s1),
                                                                      1, 16, s1), args.unroll)
        for _ in range(3):
            fg1.replay()
        extra["decode_b1"]["us_floor_step_layer_rotation"] = round(
            timer.median_loop(fg1, max(1, K // args.unroll)) / args.unroll, 3)
        del grr, rot1, fg1

        # ------------------------------------------------------------ B=4 layer rotation
        # The first four query tokens of the B=8 workload over the same
        # rotation (four units: each token's splits on two XCDs).
        q4, idx4 = q8[:4].contiguous(), idx8[:4].contiguous()
        gr4 = rotation_cycle(torch, rot, lambda kv: triton_mla_sparse_attention(q4, kv, idx4, W.SM_SCALE,
                                                                                num_kv_splits=args.splits),
                             args.unroll)
        for _ in range(3):
            gr4.replay()
        log("decode_b4 layer rotation")
        us4 = timer.median_loop(gr4, max(1, K // args.unroll)) / args.unroll
        extra["decode_b4"] = {"us_per_step_layer_rotation": round(us4, 3),
                              "gbs_layer_rotation": round(W.mla_bytes(idx4, n_rows) / (us4 * 1e-6) / 1e9, 1),
                              "workload": "tokens 0-3 of the B=8 decode workload"}
        del gr4, q4, idx4

        # ------------------------------------------------------------ paged decode B=8
        # Request-relative indices: vLLM-style conversion + attention (two
        # launches before the attention's own) against the fused call, over
        # the layer rotation (each cache seen as 4096 pages of 64 rows).
        from sparse_utils import flat_kv_row_view, triton_convert_req_index_to_global_index
        from titan_mla import triton_mla_sparse_attention_paged
        pages, qpg, idxpg, reqpg, btpg = W.paged_b8_inputs(dev, g8, cache8)
        bs_pg = pages.shape[1]
        _, stride_pg = flat_kv_row_view(pages, bs_pg)
        as_pages = lambda kv: kv.view(n_rows // bs_pg, bs_pg, W.ROW_BYTES)

        def paged_two(kv):
            flat = triton_convert_req_index_to_global_index(
                reqpg, btpg, idxpg.view(8, -1), BLOCK_SIZE=bs_pg, BLOCK_STRIDE_ROWS=stride_pg,
                NUM_TOPK_TOKENS=idxpg.shape[-1])
            return triton_mla_sparse_attention(qpg, kv, flat.view(8, 1, -1), W.SM_SCALE,
                                               num_kv_splits=args.splits)

        paged_one = lambda kv: triton_mla_sparse_attention_paged(qpg, as_pages(kv), idxpg, reqpg, btpg, W.SM_SCALE,
                                                                 num_kv_splits=args.splits)
        log("decode_b8 paged")
        gp2 = rotation(paged_two)
        gp1 = rotation(paged_one)
        for _ in range(max(1, Wm // args.unroll)):
            gp2.replay()
            gp1.replay()
        us_two = timer.median_loop(gp2, K // args.unroll) / args.unroll
        us_one = timer.median_loop(gp1, K // args.unroll) / args.unroll
        # Indexer output (top-512 pools of 4 tokens + tail): expansion +
        # conversion + attention, against the one pooled call.
        from sparse_utils import expand_pools_and_append_tail
        from titan_mla import triton_mla_sparse_attention_pooled
        pools_pg, lens_pg = W.pooled_b8_inputs(dev, g8)
        buf_pg = torch.full((8, 2176), -1, dtype=torch.int32, device=dev)

        def pooled_three(kv):
            exp = expand_pools_and_append_tail(pools_pg, lens_pg, 4)
            buf_pg[:, : exp.shape[1]].copy_(exp)
            flat = triton_convert_req_index_to_global_index(
                reqpg, btpg, buf_pg, BLOCK_SIZE=bs_pg, BLOCK_STRIDE_ROWS=stride_pg, NUM_TOPK_TOKENS=2176)
            return triton_mla_sparse_attention(qpg, kv, flat.view(8, 1, -1), W.SM_SCALE,
                                               num_kv_splits=args.splits)

        pooled_one = lambda kv: triton_mla_sparse_attention_pooled(qpg, as_pages(kv), pools_pg, lens_pg, 4, reqpg,
                                                                   btpg, W.SM_SCALE, num_kv_splits=args.splits)
        gq3 = rotation(pooled_three)
        gq1 = rotation(pooled_one)
        for _ in range(max(1, Wm // args.unroll)):
            gq3.replay()
            gq1.replay()
        us_q3 = timer.median_loop(gq3, K // args.unroll) / args.unroll
        us_q1 = timer.median_loop(gq1, K // args.unroll) / args.unroll
        extra["decode_b8_paged"] = {"us_per_step_fused": round(us_one, 3),
                                    "us_per_step_convert_then_attend": round(us_two, 3),
                                    "us_per_step_pooled_fused": round(us_q1, 3),
                                    "us_per_step_expand_convert_attend": round(us_q3, 3),
                                    "block_size": bs_pg, "context_per_request": 32768,
                                    "residency": "layer rotation (HBM)"}
        del gp1, gp2, gq1, gq3

        # ------------------------------------------------------------ MoE align
        moe = {}
        gm = W.gen(dev, W.SEED_BENCH)
        for b in (1, 2, 4, 8):
            ids = W.moe_routes(b, dev, gm)
            mg, _ = capture(torch, lambda ids=ids: titan_moe_align_small(ids), unroll=16)
            for _ in range(5):
                mg.replay()
            samples = [timer.replay_loop(mg, 100) / 16 for _ in range(5)]
            moe[f"B{b}"] = round(statistics.median(samples), 3)
            del mg
        extra["moe_align_us_per_call"] = moe
        # The dispatch floor of the same protocol: a kernel adding 1 to one
        # int32, 16 per graph.
        one = torch.zeros(1, dtype=torch.int32, device=dev)
        fg, _ = capture(torch, lambda: one.add_(1), unroll=16)
        for _ in range(5):
            fg.replay()
        extra["graph_dispatch_floor_us_per_kernel"] = round(
            statistics.median(timer.replay_loop(fg, 100) / 16 for _ in range(5)), 3)
        del fg, one
        extra["moe_align_reference_us_per_call_sm80"] = {"B1": 1.63, "B2": 1.97, "B4": 1.97, "B8": 5.07}

        # ------------------------------------------------------------ MoE W4A16 layer
        # The aligner's consumer: gate/up GEMM + SiLU, down GEMM + router
        # weights + route sum (288 experts, hidden 4096, intermediate 512).
        # "same call": one call replayed, so a small batch's experts stay in
        # the 256 MB MALL.  "layer rotation" (the decode case): 8 calls per
        # graph cycling over 4 layers' weights (4 x 1.06 GB) with fresh random
        # routes per call, as consecutive MoE layers read other experts.
        from titan_moe_w4a16 import fused_moe_w4a16, repack_w4a16, moe_w4a16_gate_up, moe_w4a16_down
        layers = []
        for li in range(4):
            lay = W.moe_w4a16_layer(dev, seed=W.SEED_BENCH + 100 + li)
            layers.append(repack_w4a16(lay["w13_packed"], lay["w13_scale"]) +
                          repack_w4a16(lay["w2_packed"], lay["w2_scale"]))
            del lay
        moew = {}
        for b in (1, 2, 4, 8):
            gmw = W.gen(dev, W.SEED_BENCH + b)
            calls = []
            for i in range(MOE_ROT_CALLS):
                xm, idm, twm = W.moe_w4a16_inputs(b, dev, gmw)
                calls.append((xm, idm, twm, layers[i % 4]))
            one = lambda c=calls[0]: fused_moe_w4a16(c[0], c[3][0], c[3][2], c[3][1], c[3][3], c[2], c[1])
            rot_moe = lambda: [fused_moe_w4a16(c[0], c[3][0], c[3][2], c[3][1], c[3][3], c[2], c[1]) for c in calls]
            gw, _ = capture(torch, one, args.unroll)
            gr, _ = capture(torch, rot_moe, 1)
            for _ in range(3):
                gw.replay()
                gr.replay()
            log(f"moe w4a16 B={b}")
            us_same = timer.replay_loop(gw, max(2, K // args.unroll // 2)) / args.unroll
            us_rot = timer.replay_loop(gr, max(4, K // 8)) / len(calls)
            del gw, gr
            # The aligner's cost per layer: the fused layer aligns inside its
            # gate/up kernel; the same layer as three launches (the aligner
            # kernel, gate/up over its blocks, down), and as two launches
            # over alignments computed beforehand (no alignment cost at all).
            aligned = [titan_moe_align_small(c[1]) for c in calls]

            def staged(c, al=None):
                al = al if al is not None else titan_moe_align_small(c[1])
                act = moe_w4a16_gate_up(c[0], c[3][0], c[3][1], al[0], al[1])
                return moe_w4a16_down(act, c[3][2], c[3][3], c[2], c[1])
            gsep, _ = capture(torch, lambda: [staged(c) for c in calls], 1)
            gpre, _ = capture(torch, lambda: [staged(c, al) for c, al in zip(calls, aligned)], 1)
            for _ in range(3):
                gsep.replay()
                gpre.replay()
            us_sep = timer.replay_loop(gsep, max(4, K // 8)) / len(calls)
            us_pre = timer.replay_loop(gpre, max(4, K // 8)) / len(calls)
            del gsep, gpre, aligned
            mb = statistics.mean(W.moe_w4a16_bytes(c[1], b) for c in calls)
            moew[f"B{b}"] = {"us_per_call_same_call": round(us_same, 2),
                             "us_per_call_layer_rotation": round(us_rot, 2),
                             "us_per_call_layer_rotation_align_kernel_then_gemms": round(us_sep, 2),
                             "us_per_call_layer_rotation_prealigned_gemms": round(us_pre, 2),
                             "align_cost_in_fused_layer_us": round(us_rot - us_pre, 2),
                             "align_cost_as_separate_kernel_us": round(us_sep - us_pre, 2),
                             "algorithmic_bytes_mean": round(mb),
                             "gbs_layer_rotation": round(mb / (us_rot * 1e-6) / 1e9, 1),
                             "hbm_frac_layer_rotation": round(mb / (us_rot * 1e-6) / 1e9 / HBM_PEAK_GBS, 3)}
            del calls
        extra["moe_w4a16_layer"] = moew

        # ------------------------------------------------------------ sparse indexer (decode)
        # FP8 paged MQA logits of each request's 65536 pools (262144-token
        # context, 4 tokens per pool, 32 heads, 64-pool pages), then the
        # top-512 pools per request.  "warm": one call replayed (its pool
        # cache stays in the 256 MB MALL); "rotation" (the decode case, each
        # layer reading its own cache): calls cycling over enough caches
        # (> 512 MB) that every call reads its cache from HBM.
        from sparse_indexer import fp8_paged_mqa_logits, indexer_topk, indexer_decode_pool_topk
        idx = {}
        for b, n_caches in ((1, 64), (8, 8)):
            gi = W.gen(dev, W.SEED_BENCH + 200 + b)
            sets = [W.indexer_decode_inputs(dev, gi, batch=b) for _ in range(n_caches)]
            q_i, cache_i, w_i, lens_i, bt_i, pools = sets[0]
            logits_i = fp8_paged_mqa_logits(q_i, cache_i, w_i, lens_i, bt_i, pools, clean_logits=False)
            row = {}
            log(f"indexer decode B={b}")
            for name, fn in (("logits", lambda s: fp8_paged_mqa_logits(*s, clean_logits=False)),
                             ("logits_plus_topk", lambda s: indexer_decode_pool_topk(*s))):
                gg, _ = capture(torch, lambda: fn(sets[0]), args.unroll)
                gr, _ = capture(torch, lambda: [fn(s) for s in sets], 1)
                for _ in range(3):
                    gg.replay()
                    gr.replay()
                row[f"us_{name}_warm"] = round(timer.replay_loop(gg, max(2, K // args.unroll // 2)) / args.unroll, 2)
                row[f"us_{name}_rotation"] = round(timer.replay_loop(gr, 10) / n_caches, 2)
                del gg, gr
            gt, _ = capture(torch, lambda: indexer_topk(logits_i, lens_i, W.INDEX_TOPK_POOLS), args.unroll)
            gt.replay()
            row["us_topk"] = round(timer.replay_loop(gt, max(2, K // args.unroll // 2)) / args.unroll, 2)
            del gt
            nb = W.indexer_bytes(lens_i)
            row["logits_algorithmic_bytes"] = nb
            for tag in ("warm", "rotation"):
                gbs = nb / (row[f"us_logits_{tag}"] * 1e-6) / 1e9
                row[f"logits_gbs_{tag}"] = round(gbs, 1)
                row[f"logits_hbm_frac_{tag}"] = round(gbs / HBM_PEAK_GBS, 3)
            idx[f"B{b}"] = row
            del sets, q_i, cache_i, w_i, lens_i, bt_i, logits_i
        extra["indexer_decode"] = idx

        # ------------------------------------------------------------ one decode layer's path, B=8
        # The path's rows composed as one layer of a B=8 decode step (8
        # requests at 262144 tokens sharing one 262144-row cache, the headline
        # shape): the 8 new latents written (store_int8), the indexer's
        # logits + top-512 pools, the pooled attention (expansion, page
        # mapping and split-KV in one launch, then the merge) and the fused
        # W4A16 MoE layer.  4 layers of their own caches, pool caches and
        # expert weights cycled in a graph of 16 steps (≈ 1.1 GB read per
        # cycle of 4: HBM), against the same components' graphs alone over the
        # same layers.
        from titan_mla import triton_mla_sparse_attention_pooled
        gl = W.gen(dev, W.SEED_BENCH + 500)
        lay_path = []
        for li in range(4):
            _, xl, cl, sl = W.decode_cache(dev, seed=W.SEED_BENCH + 500 + li, dist="t3")
            store_int8(xl, cl, sl)
            del xl, sl
            iset = W.indexer_decode_inputs(dev, gl, batch=8)
            xm, idm, twm = W.moe_w4a16_inputs(8, dev, gl)
            lay_path.append((cl, iset, (xm, idm, twm, layers[li])))
        pages = n_rows // W.BLOCK
        bt_path = torch.arange(pages, dtype=torch.int32, device=dev).repeat(8, 1).contiguous()
        req_path = torch.arange(8, dtype=torch.int32, device=dev)
        q_path = torch.randn(8, 16, 512, generator=gl, device=dev).to(torch.bfloat16)
        x_new = torch.randn(8, 512, generator=gl, device=dev).to(torch.bfloat16)
        slots_path = torch.randperm(n_rows, generator=gl, device=dev)[:8]

        def write(lp):
            store_int8(x_new, lp[0], slots_path)

        def index(lp):
            return indexer_decode_pool_topk(*lp[1])

        def attend(lp, pools_l):
            seq_l = lp[1][3] * W.INDEX_KPOOL          # complete pools: no tail
            return triton_mla_sparse_attention_pooled(q_path, lp[0], pools_l, seq_l, W.INDEX_KPOOL, req_path,
                                                      bt_path, W.SM_SCALE, topk=W.TOPK)

        def moe(lp):
            c = lp[2]
            return fused_moe_w4a16(c[0], c[3][0], c[3][2], c[3][1], c[3][3], c[2], c[1])

        pools_pre = [index(lp) for lp in lay_path]      # the attention-alone graph's inputs
        cyc = 4                                         # the 4 layers 4 times: 16 steps per graph
        parts = {"store_int8": lambda: [write(lp) for _ in range(cyc) for lp in lay_path],
                 "indexer_logits_topk": lambda: [index(lp) for _ in range(cyc) for lp in lay_path],
                 "pooled_attention": lambda: [attend(lp, p) for _ in range(cyc) for lp, p in zip(lay_path, pools_pre)],
                 "moe_w4a16_layer": lambda: [moe(lp) for _ in range(cyc) for lp in lay_path],
                 "layer": lambda: [(write(lp), attend(lp, index(lp)), moe(lp)) for _ in range(cyc) for lp in lay_path]}
        path = {}
        log("decode layer path B=8 (write + indexer + pooled attention + MoE), 4 layers")
        for name, fn in parts.items():
            gpth, _ = capture(torch, fn, 1)
            for _ in range(3):
                gpth.replay()
            path[f"us_{name}"] = round(timer.replay_loop(gpth, max(4, K // 8)) / (cyc * len(lay_path)), 2)
            del gpth
        path["us_sum_of_parts"] = round(sum(v for k, v in path.items() if k != "us_layer"), 2)
        path["what"] = ("per layer, B=8 decode over 262144-token contexts: store_int8 of 8 rows, indexer logits "
                        "over 65536 pools + top-512, pooled sparse MLA (2176 slots), fused W4A16 MoE; 4 layers "
                        "cycled 4 times in one graph of 16 steps, each component alone the same way")
        extra["decode_layer_path_b8"] = path
        del lay_path, pools_pre, layers

        # ------------------------------------------------------------ sparse indexer (prefill shape)
        # The reference's TP4 prefill indexer benchmark, replicated branch on
        # one GPU (docs/measurements.json:3196-3201: 20.632 ms wall median for
        # 2048 rows): 2048 query rows at the end of a 262144-token context,
        # logits over the complete pools before each row (65536 pools) and the
        # top 512 per row.  Three calls per graph, median of 5 samples.
        gi = W.gen(dev, W.SEED_BENCH + 2048)
        qpi, cpi, wpi, lpi, bpi, npi = W.indexer_prefill_inputs(dev, gi)
        pre_fn = lambda: indexer_topk(fp8_paged_mqa_logits(qpi, cpi, wpi, lpi, bpi, npi, clean_logits=False), lpi,
                                      W.INDEX_TOPK_POOLS)
        gpi, _ = capture(torch, pre_fn, 3)
        gpi.replay()
        log("indexer prefill shape (2048 rows)")
        us_pi = timer.median_loop(gpi, 2) / 3
        del gpi
        glo, _ = capture(torch, lambda: fp8_paged_mqa_logits(qpi, cpi, wpi, lpi, bpi, npi, clean_logits=False), 3)
        glo.replay()
        us_plo = timer.median_loop(glo, 2) / 3
        del glo
        fl = W.indexer_flops(lpi)
        extra["indexer_prefill_2048_rows"] = {"ms_logits_plus_topk": round(us_pi / 1e3, 4),
                                              "ms_logits": round(us_plo / 1e3, 4),
                                              "logits_fp8_tflops": round(fl / (us_plo * 1e-6) / 1e12, 1),
                                              "logits_mfma_frac": round(fl / (us_plo * 1e-6) / FP8_PEAK_FLOPS, 3),
                                              "reference_ms_replicated_sm80": 20.632,
                                              "speedup_vs_reference": round(20.632e3 / us_pi, 1),
                                              "pools": npi, "rows": int(lpi.numel()), "heads": W.INDEX_HEADS}
        del qpi, cpi, wpi, lpi, bpi

        # ------------------------------------------------------------ prefill-shaped
        # T=2048 tokens, one split.  warm: one cache replayed (138 MB, MALL-
        # resident); rotation: consecutive calls over 3 caches (415 MB, read
        # from HBM).
        qp, idxp, new_rows, pslots = W.prefill_inputs(dev, g8)
        pg, _ = capture(torch, lambda: triton_mla_sparse_attention(qp, kv8, idxp, W.SM_SCALE), 3)
        pg.replay()
        log("prefill T=2048")
        us_p = timer.median_loop(pg, 3) / 3
        del pg
        pgr, _ = capture(torch, lambda: [triton_mla_sparse_attention(qp, c, idxp, W.SM_SCALE) for c in rot[:3]])
        pgr.replay()
        us_pr = timer.median_loop(pgr, 3) / 3
        del pgr
        bytes_p = W.mla_bytes(idxp, n_rows)
        flops_p = W.mla_flops(idxp, n_rows)
        extra["prefill_t2048"] = {"us_per_call_warm": round(us_p, 1), "us_per_call_rotation": round(us_pr, 1),
                                  "algorithmic_bytes": bytes_p,
                                  "gbs_warm": round(bytes_p / (us_p * 1e-6) / 1e9, 1),
                                  "gbs_rotation": round(bytes_p / (us_pr * 1e-6) / 1e9, 1),
                                  "hbm_frac_rotation": round(bytes_p / (us_pr * 1e-6) / 1e9 / HBM_PEAK_GBS, 3),
                                  "tflops_warm": round(flops_p / (us_p * 1e-6) / 1e12, 2)}
        # The same call in request-relative form (a vLLM-style paged prefill):
        # one request whose 262144 tokens sit in 4096 pages of 64 rows at
        # random places, the indices positions within the request; the block
        # table lookup runs inside the attention's gather.
        from titan_mla import triton_mla_sparse_attention_paged
        pp_pages = cache8.view(n_rows // 64, 64, W.ROW_BYTES)
        pp_bt = torch.randperm(pp_pages.shape[0], generator=g8, device=dev).to(torch.int32)[None, :].contiguous()
        pp_req = torch.zeros(qp.shape[0], dtype=torch.int32, device=dev)
        ppg, _ = capture(torch, lambda: triton_mla_sparse_attention_paged(qp, pp_pages, idxp, pp_req, pp_bt,
                                                                           W.SM_SCALE), 3)
        ppg.replay()
        us_pp = timer.median_loop(ppg, 3) / 3
        del ppg
        extra["prefill_t2048"]["us_per_call_paged_warm"] = round(us_pp, 1)
        # the prefill-shaped call's write: 2048 rows into randperm slots,
        # `unroll` calls per graph (one call per graph would time the graph
        # launch, ~15 us, not the kernel's ~3 us)
        c5 = torch.zeros_like(cache8)
        wpg, _ = capture(torch, lambda: store_int8(new_rows, c5, pslots), args.unroll)
        wpg.replay()
        us_ws = timer.median_loop(wpg, max(2, K // args.unroll)) / args.unroll
        extra["store_int8_2048_scattered"] = {"us_per_call": round(us_ws, 2),
                                              "gbs": round(W.writer_bytes(2048) / (us_ws * 1e-6) / 1e9, 1),
                                              "calls_per_graph": args.unroll}
        del wpg, c5

        # ------------------------------------------------------------ CPU baseline
        if not args.no_cpu:
            # The C oracle on this host's cores (OpenMP over tokens / rows), each
            # configuration's own inputs, and 1 thread beside it; 3 warm-ups, the
            # median of 5 samples of at least --cpu-sample-s seconds.
            import oracle
            oracle.build()
            threads = oracle.default_threads()
            ms = args.cpu_sample_s
            u16 = lambda t: t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
            rows8 = cache8.view(torch.uint8).cpu().numpy().reshape(-1, W.ROW_BYTES)
            rows1 = cache1.view(torch.uint8).cpu().numpy().reshape(-1, W.ROW_BYTES)
            cfgs = {}

            def both(name, fn1, nbytes, unit_note, gpu_us, per_call=1, single_threaded=False):
                log(f"CPU baseline {name}")
                row = {}
                if not single_threaded:
                    us_n = cpu_time(lambda: fn1(threads), ms, per_call)
                    row.update(us_per_call=round(us_n, 1), threads=threads,
                               gbs=round(nbytes / (us_n * 1e-6) / 1e9, 3) if nbytes else None)
                us_1 = cpu_time(lambda: fn1(1), ms, per_call)
                row.update(us_per_call_1thread=round(us_1, 2 if us_1 < 100 else 1),
                           gbs_1thread=round(nbytes / (us_1 * 1e-6) / 1e9, 4) if nbytes else None,
                           gpu_us_per_call=gpu_us, what=unit_note)
                cfgs[name] = row
                return row
            # the writer: 262144 N(0,1) rows (the same seeded latents as the GPU's)
            _, xw, _, _ = W.decode_cache(dev, seed=W.SEED_BENCH + 1, dist="normal")
            xw_u16 = u16(xw)
            del xw
            both("store_int8_262144_normal", lambda t: oracle.quantize_rows(xw_u16, nthreads=t), wb,
                 "store_int8 of 262144 rows into 528-byte rows", extra["store_int8_262144"]["us_per_call_hbm_rotation"])
            del xw_u16
            # B=1 over the N(0,1) cache
            q1n, ix1n = u16(q1), idx1.cpu().numpy()
            both("decode_b1_normal", lambda t: oracle.sparse_mla(q1n, rows1, ix1n, W.SM_SCALE, n_splits=s1, nthreads=t),
                 bytes1, "one B=1 sparse MLA step", extra["decode_b1"]["us_per_step_layer_rotation"])
            # B=8 over the Student-t cache (the headline)
            qn, ixn = u16(q8), idx8.cpu().numpy()
            r8 = both("decode_b8_t3", lambda t: oracle.sparse_mla(qn, rows8, ixn, W.SM_SCALE, n_splits=s8, nthreads=t),
                      bytes8, "one B=8 sparse MLA step", round(us8, 3))
            # a sample of 64 of the prefill-shaped call's 2048 tokens
            pick = np.unique(np.linspace(0, qp.shape[0] - 1, 64).astype(np.int64))
            qpn, ixpn = u16(qp)[pick], idxp.cpu().numpy()[pick]
            pbytes = W.mla_bytes(idxp[torch.as_tensor(pick, device=dev)], n_rows)
            rp = both("prefill_64_of_2048_tokens",
                      lambda t: oracle.sparse_mla(qpn, rows8, ixpn, W.SM_SCALE, n_splits=1, nthreads=t),
                      pbytes, "64 evenly spaced tokens of the T=2048 call (one split each)",
                      round(extra["prefill_t2048"]["us_per_call_rotation"] * len(pick) / qp.shape[0], 2))
            rp["us_per_call_all_2048_tokens_est"] = round(rp["us_per_call"] * qp.shape[0] / len(pick))
            # MoE align B1..8 (the reference's CPU algorithm: a stable
            # counting sort over the 288 experts; single-threaded), 1000 calls
            # per timed call through ctypes
            gm2 = W.gen(dev, W.SEED_BENCH)
            for b in (1, 2, 4, 8):
                ids_b = W.moe_routes(b, dev, gm2).cpu().numpy()
                both(f"moe_align_B{b}", lambda t, ids_b=ids_b: oracle.moe_align_repeat(ids_b, 1000), 0,
                     "one align call (1000 per timed call)", extra["moe_align_us_per_call"][f"B{b}"], per_call=1000,
                     single_threaded=True)
            cfgs["host"] = {"threads_used": threads, "os_cpu_count": os.cpu_count(),
                            "affinity_cpus": len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None,
                            "cpu_model": cpu_model(),
                            "timing": f"C oracle (-O2, OpenMP), 3 warm-ups, median of 5 samples of >= {ms:g} s each"}
            extra["cpu_baseline_configs"] = cfgs
            cpu = {"value": r8["gbs"], "unit": "GB/s", "cores": threads, "kind": "port",
                   "sample": f"the full decode_b8 workload (one B=8 sparse MLA step over the 262144-row cache): "
                             f"the C oracle on {threads} threads, 3 warm-ups, median of 5 samples of >= {ms:g} s",
                   "us_per_step": r8["us_per_call"], "us_per_step_1thread": r8["us_per_call_1thread"],
                   "os_cpu_count": os.cpu_count(), "affinity_cpus": cfgs["host"]["affinity_cpus"]}

            # The widened rows' CPU paths (the numpy oracle: float64 reference
            # arithmetic, one call each) beside their GPU figures above.
            rows_cpu = {}
            lay = W.moe_w4a16_layer(dev, seed=W.SEED_BENCH + 100)
            bits = lambda t: t.view(torch.int16).cpu().numpy().view(np.uint16)
            w13n, s13n = lay["w13_packed"].cpu().numpy(), bits(lay["w13_scale"])
            w2n, s2n = lay["w2_packed"].cpu().numpy(), bits(lay["w2_scale"])
            del lay
            for b in (1, 8):
                xm, idm, twm = W.moe_w4a16_inputs(b, dev, W.gen(dev, W.SEED_BENCH + b))
                log(f"CPU oracle: W4A16 MoE layer B={b}")
                t0 = time.perf_counter()
                oracle.moe_w4a16(bits(xm), w13n, s13n, w2n, s2n, twm.cpu().numpy(), idm.cpu().numpy())
                us_c = (time.perf_counter() - t0) * 1e6
                gpu_us = extra["moe_w4a16_layer"][f"B{b}"]["us_per_call_layer_rotation"]
                rows_cpu[f"moe_w4a16_layer_B{b}"] = {"cpu_us": round(us_c), "gpu_us": gpu_us,
                                                     "speedup": round(us_c / gpu_us)}
            del w13n, s13n, w2n, s2n
            gi = W.gen(dev, W.SEED_BENCH + 201)
            q_i, cache_i, w_i, lens_i, bt_i, pools = W.indexer_decode_inputs(dev, gi, batch=1)
            page = cache_i.stride(0)
            pages = torch.as_strided(cache_i, (cache_i.shape[0], page), (page, 1)).cpu().numpy()
            log("CPU oracle: indexer logits + top-512 B=1")
            t0 = time.perf_counter()
            lg = oracle.fp8_paged_mqa_logits(q_i.view(torch.uint8).cpu().numpy().reshape(1, -1, 128), pages,
                                             cache_i.shape[1], w_i.cpu().numpy(), lens_i.cpu().numpy(),
                                             bt_i.cpu().numpy(), pools, clean=False)
            oracle.indexer_topk(lg, lens_i.cpu().numpy(), W.INDEX_TOPK_POOLS)
            us_c = (time.perf_counter() - t0) * 1e6
            gpu_us = extra["indexer_decode"]["B1"]["us_logits_plus_topk_rotation"]
            rows_cpu["indexer_logits_plus_topk_B1"] = {"cpu_us": round(us_c), "gpu_us": gpu_us,
                                                       "speedup": round(us_c / gpu_us)}
            del pages, lg, q_i, cache_i
            rows_cpu["note"] = ("numpy oracle (float64 arithmetic, library threads as configured), one call; "
                                "GPU figures: layer rotation / cache rotation")
            extra["cpu_oracle_rows"] = rows_cpu

    # dominant kernel: sparse_mla_kernel (split attention); algorithmic bytes of
    # the step over its event-timed average duration in the same HBM-resident
    # rotation.  traffic: measured HBM-side bytes per dispatch (rocprofv3
    # FETCH_SIZE + WRITE_SIZE, copy-calibrated), keyed by kernel and grid
    # (workgroups x threads): a grid with no committed measurement gives null
    # and says so.
    ach = bytes8 / (us8_kernel * 1e-6) / 1e9
    traffic, traffic_note = None, None
    key = f"sparse_mla_kernel@{s8 * 8 * split_kernel_threads(W.TOPK, s8)}"
    tf = ROOT / "profiles" / "hbm_bytes_per_dispatch.json"
    d = json.loads(tf.read_text())["per_dispatch"].get(key) if tf.exists() else None
    if d:
        traffic = d["fetch_bytes"] + d["write_bytes"]
        traffic_note = (f"{tf.relative_to(ROOT)} [{key}]: FETCH_SIZE + WRITE_SIZE per dispatch, "
                        f"{d.get('run', '')}; measured at commit {d.get('commit', 'unrecorded')}")
    else:
        traffic_note = f"no HBM byte measurement for {key} in {tf.relative_to(ROOT)}"
        log(f"WARNING: roofline.traffic is null: {traffic_note}")
        traffic_note = "null: " + traffic_note
    roofline = {"bound": "hbm", "kernel": "sparse_mla_kernel", "achieved": round(ach, 1),
                "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
                "traffic": traffic, "algorithmic_bytes": bytes8,
                "avg_kernel_us": round(us8_kernel, 3),
                "timing": f"median of {n_samples} samples of {K} launches, HBM-resident (layer rotation)"}
    if traffic_note:
        roofline["traffic_source"] = traffic_note
    roofline["profile"] = ("profiles/sparse_mla_decode_b8_split_rotation.txt: rocprofv3 kernel trace of this "
                           "region (bench.py --case decode_b8_split --rotate 256)")
    if cpu is not None:
        cpu["cpu_model"] = cpu_model()
    line = {
        "metric": METRIC,
        "value": round(gbs8, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": Wm,
        "ms_per_step": round(us8 / 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "decode_b8: sparse NoPE MLA decode, B=8, 16 heads, 262144-row INT8 cache, "
                               "2176 indices/query (locality-biased, 0-256 trailing pads), Student-t latents",
                   "batch": 8, "context": n_rows, "topk": W.TOPK, "heads": 16, "num_kv_splits": s8,
                   "timing": f"HIP graph replay, {args.unroll} steps per graph, median of {n_samples} samples "
                             f"of {K} steps",
                   "residency": f"HBM: consecutive steps cycle over {len(rot)} caches of 262144 rows "
                                f"({len(rot) * bytes8 / 1e6:.0f} MB of rows touched per cycle > the 256 MB "
                                "MALL); "
                                "the warm (MALL-resident) figure is extra.decode_b8.us_per_step_warm"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "device": {"name": props.name, "cus": cu},
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
