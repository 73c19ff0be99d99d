"""Seeded synthetic inputs for the decode hot path's benchmark configurations.

Shared by tests/ and bench.py.  Everything is generated on the target device
with a torch.Generator, so the same seed gives the same tensors on every run
of the same build.  Seeds follow the reference's choices: 20260910 for
fixtures (tests/verify_mla.py:107) and 37 for benchmarks (benchmarks/mla.py:27).

Configurations (sizes as in the benchmark definition):
  writer_small   store_int8 of 16384 N(0,1) rows into [64, 256, 528], slots arange;
                 decode B=1 with 2176 indices uniform in [0, 16384), last 128 = -1
  moe_small      routes [B, 8], 8 distinct experts per token from 288, B in {1,2,4,8}
  decode_b1      262144 N(0,1) rows into [1024, 256, 528]; q [1, 16, 512];
                 2048 indices uniform in [0, 262144) then 128 x -1
  decode_b8      the same cache from Student-t(3) x 0.5 latents; q [8, 16, 512];
                 per batch 0..256 trailing -1 pads, half of the valid indices in
                 the last 4096 positions, half uniform
  prefill_t2048  q [2048, 16, 512]; token t at position 260096 + t with 2176
                 indices <= its position (half within 4096 behind it, half
                 uniform); store_int8 of 2048 new rows to a random permutation
                 of slots
"""
from __future__ import annotations

import math

import torch

SEED_FIXTURE = 20260910
SEED_BENCH = 37
LATENT = 512
ROW_BYTES = 528
BLOCK = 256
TOPK = 2176
HEADS = 16
SM_SCALE = 512 ** -0.5


def gen(device, seed):
    return torch.Generator(device=device).manual_seed(seed)


def student_t3(shape, g, device, dtype=torch.float32):
    """Student-t with 3 degrees of freedom: z / sqrt(chi2_3 / 3)."""
    z = torch.randn(shape, generator=g, device=device, dtype=dtype)
    chi = torch.zeros(shape, device=device, dtype=dtype)
    for _ in range(3):
        chi += torch.randn(shape, generator=g, device=device, dtype=dtype) ** 2
    return z / torch.sqrt(chi / 3)


def latents(n, device, g, dist="normal", chunk=65536):
    out = torch.empty(n, LATENT, device=device, dtype=torch.bfloat16)
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        if dist == "normal":
            out[s:e] = torch.randn(e - s, LATENT, generator=g, device=device)
        else:
            out[s:e] = student_t3((e - s, LATENT), g, device) * 0.5
    return out


def empty_cache(n_rows, device):
    assert n_rows % BLOCK == 0
    return torch.zeros(n_rows // BLOCK, BLOCK, ROW_BYTES, device=device, dtype=torch.int8)


def uniform_indices(batch, n_rows, valid, device, g):
    idx = torch.randint(n_rows, (batch, 1, TOPK), generator=g, device=device, dtype=torch.int32)
    idx[:, :, valid:] = -1
    return idx


def local_biased_indices(batch, n_rows, device, g, max_pads=256, window=4096, positions=None):
    """Per row b: pads_b ~ U{0..max_pads} trailing -1; of the valid entries half
    fall in [pos_b - window + 1, pos_b] and half uniform in [0, pos_b]
    (pos_b = n_rows - 1 unless positions are given), in random order."""
    idx = torch.full((batch, 1, TOPK), -1, device=device, dtype=torch.int32)
    pads = torch.randint(0, max_pads + 1, (batch,), generator=g, device=device)
    pos = (torch.full((batch,), n_rows - 1, device=device, dtype=torch.int64)
           if positions is None else positions.to(torch.int64))
    lo = (pos - window + 1).clamp_min(0)
    u1 = torch.rand(batch, TOPK, generator=g, device=device, dtype=torch.float64)
    u2 = torch.rand(batch, TOPK, generator=g, device=device, dtype=torch.float64)
    pick_local = torch.rand(batch, TOPK, generator=g, device=device) < 0.5
    local = lo[:, None] + torch.floor(u1 * (pos - lo + 1)[:, None].to(torch.float64)).to(torch.int64)
    unif = torch.floor(u2 * (pos + 1)[:, None].to(torch.float64)).to(torch.int64)
    vals = torch.where(pick_local, local, unif).to(torch.int32)
    keep = torch.arange(TOPK, device=device)[None, :] < (TOPK - pads)[:, None]
    idx[:, 0, :] = torch.where(keep, vals, torch.full_like(vals, -1))
    return idx


def writer_small(device, seed=SEED_BENCH):
    g = gen(device, seed)
    n = 16384
    x = latents(n, device, g)
    cache = empty_cache(n, device)
    slots = torch.arange(n, device=device, dtype=torch.int64)
    q = torch.randn(1, HEADS, LATENT, generator=g, device=device).to(torch.bfloat16)
    idx = uniform_indices(1, n, TOPK - 128, device, g)
    return dict(x=x, cache=cache, slots=slots, q=q, idx=idx, n_rows=n)


def decode_cache(device, seed=SEED_BENCH, dist="normal", n_rows=262144):
    g = gen(device, seed)
    x = latents(n_rows, device, g, dist)
    cache = empty_cache(n_rows, device)
    slots = torch.arange(n_rows, device=device, dtype=torch.int64)
    return g, x, cache, slots


def decode_b1_inputs(device, g, n_rows=262144):
    q = torch.randn(1, HEADS, LATENT, generator=g, device=device).to(torch.bfloat16)
    idx = uniform_indices(1, n_rows, 2048, device, g)
    return q, idx


def decode_b8_inputs(device, g, n_rows=262144):
    q = torch.randn(8, HEADS, LATENT, generator=g, device=device).to(torch.bfloat16)
    idx = local_biased_indices(8, n_rows, device, g)
    return q, idx


def paged_b8_inputs(device, g, cache, block_size=64, context=32768):
    """The decode_b8 shape in request-relative form: the 262144-row cache seen
    as pages of block_size rows, 8 requests of `context` tokens each owning a
    random set of pages (block table [8, context / block_size]), one query
    token per request, indices request-relative positions (locality-biased
    toward the request's end, 0..256 trailing pads)."""
    n_rows = cache.shape[0] * cache.shape[1]
    pages = cache.view(n_rows // block_size, block_size, ROW_BYTES)
    per_req = context // block_size
    bt = torch.randperm(pages.shape[0], generator=g, device=device)[: 8 * per_req]
    bt = bt.view(8, per_req).to(torch.int32).contiguous()
    req = torch.arange(8, device=device, dtype=torch.int32)
    q = torch.randn(8, HEADS, LATENT, generator=g, device=device).to(torch.bfloat16)
    idx = local_biased_indices(8, context, device, g)
    return pages, q, idx, req, bt


def pooled_b8_inputs(device, g, context=32768, pool_size=4, num_pools=512):
    """Indexer output for the paged B=8 decode: per request, 512 distinct
    top pools of 4 tokens (half among the last 1024 pools, half anywhere) and
    the query's sequence length (context - 1: a 3-token tail pool)."""
    n_pools = context // pool_size
    rows = []
    for _ in range(8):
        recent = n_pools - 1024 + torch.randperm(1024, generator=g, device=device)[: num_pools // 2]
        rest = torch.randperm(n_pools - 1024, generator=g, device=device)[: num_pools // 2]
        rows.append(torch.cat([recent, rest])[torch.randperm(num_pools, generator=g, device=device)])
    pools = torch.stack(rows).to(torch.int32).contiguous()
    seq_lens = torch.full((8,), context - 1, device=device, dtype=torch.int32)
    return pools, seq_lens


def prefill_inputs(device, g, n_rows=262144, tokens=2048):
    q = torch.randn(tokens, HEADS, LATENT, generator=g, device=device).to(torch.bfloat16)
    pos = n_rows - tokens + torch.arange(tokens, device=device)
    idx = local_biased_indices(tokens, n_rows, device, g, max_pads=0, positions=pos)
    new_rows = torch.randn(tokens, LATENT, generator=g, device=device).to(torch.bfloat16)
    slots = torch.randperm(n_rows, generator=g, device=device)[:tokens]
    return q, idx, new_rows, slots


def moe_routes(batch, device, g, dtype=torch.int32):
    """8 distinct experts per token drawn uniformly from 288."""
    keys = torch.rand(batch, 288, generator=g, device=device)
    return keys.argsort(dim=1)[:, :8].to(dtype).contiguous()


# ----------------------------------------------------------------- MoE W4A16 layer

MOE_EXPERTS = 288
MOE_HIDDEN = 4096
MOE_INTER = 512      # per-rank expert intermediate size under TP4
MOE_TOPK = 8


def moe_w4a16_layer(device, seed=SEED_BENCH, experts=MOE_EXPERTS, hidden=MOE_HIDDEN, inter=MOE_INTER):
    """Random-init W4A16 group-32 expert weights at the GLM-5.3 TP4 shape in
    the checkpoint packing (int32 [E, n_out, K/8], bf16 scales [E, n_out,
    K/32]): uniform 4-bit codes (std of q - 8 = 4.61) and scales drawn around
    1 / (4.61 sqrt(K)) for W13 and 1 / (0.6 * 4.61 sqrt(N)) for W2, so gate,
    up and the down outputs have unit scale for unit-normal inputs."""
    g = gen(device, seed)
    codes = lambda n_out, k: torch.randint(0, 256, (experts, n_out, k // 2), generator=g, device=device,
                                           dtype=torch.uint8).view(torch.int32)
    scale = lambda n_out, k, base: ((torch.rand(experts, n_out, k // 32, generator=g, device=device) + 0.5)
                                    * base).to(torch.bfloat16)
    return {
        "w13_packed": codes(2 * inter, hidden),
        "w13_scale": scale(2 * inter, hidden, 1.0 / (4.61 * math.sqrt(hidden))),
        "w2_packed": codes(hidden, inter),
        "w2_scale": scale(hidden, inter, 1.0 / (0.6 * 4.61 * math.sqrt(inter))),
    }


def moe_w4a16_inputs(batch, device, g, hidden=MOE_HIDDEN, ids=None):
    """Decode tokens for the MoE layer: unit-normal bf16 hidden states, 8
    distinct experts per token (unless ids are given) and softmax router
    weights (fp32, each row sums to 1)."""
    x = torch.randn(batch, hidden, generator=g, device=device).to(torch.bfloat16)
    if ids is None:
        ids = moe_routes(batch, device, g)
    logits = torch.randn(batch, MOE_TOPK, generator=g, device=device)
    return x, ids, torch.softmax(logits, dim=1).contiguous()


def moe_w4a16_bytes(ids: torch.Tensor, batch: int, experts=MOE_EXPERTS, hidden=MOE_HIDDEN,
                    inter=MOE_INTER) -> int:
    """Algorithmic bytes of one MoE layer call: the codes and scales of
    every distinct expert the routes use (W13 and W2), the hidden states in
    and the output out.  The c2 intermediate is implementation traffic."""
    e = ids.flatten().long()
    distinct = int(torch.unique(e[(e >= 0) & (e < experts)]).numel())
    per_expert = (2 * inter * hidden + hidden * inter) // 2 + (2 * inter * hidden + hidden * inter) // 32 * 2
    return distinct * per_expert + 2 * batch * hidden * 2


# ----------------------------------------------------------------- sparse indexer (decode scoring)

INDEX_HEADS = 32
INDEX_DIM = 128
INDEX_KPOOL = 4
INDEX_TOPK_POOLS = 512


def indexer_cache(device, g, num_pools, block_size=64, page_pad=0):
    """Pool keys in DeepGEMM's fused FP8 layout: unit-normal keys quantised
    per key to E4M3 with s = amax / 448.  Returns (cache uint8 [num_blocks,
    block_size, 1, 132] (page stride padded by page_pad bytes), num_blocks)."""
    nb = (num_pools + block_size - 1) // block_size
    k = torch.randn(nb * block_size, INDEX_DIM, generator=g, device=device)
    s = (k.abs().amax(dim=1, keepdim=True) / 448.0).clamp(min=1e-12)
    codes = (k / s).to(torch.float8_e4m3fn).view(torch.uint8).view(nb, block_size * INDEX_DIM)
    page = block_size * (INDEX_DIM + 4) + page_pad
    flat = torch.zeros(nb, page, dtype=torch.uint8, device=device)
    flat[:, : block_size * INDEX_DIM] = codes
    flat[:, block_size * INDEX_DIM: block_size * (INDEX_DIM + 4)] = s.view(nb, block_size).contiguous().view(torch.uint8)
    cache = torch.as_strided(flat, (nb, block_size, 1, INDEX_DIM + 4), (page, INDEX_DIM + 4, INDEX_DIM + 4, 1))
    return cache, nb


def indexer_decode_inputs(device, g, batch=8, context=262144, block_size=64, heads=INDEX_HEADS):
    """Decode indexer step at the full context: each request owns
    context / 4 pools in its own randomly placed pages.  Returns (q fp8 [B,
    1, H, 128], cache, weights fp32 [B, H], context_lens int32 [B] (pools),
    block_table int32 [B, max_blocks], max_model_len (pools))."""
    pools = context // INDEX_KPOOL
    per_req = (pools + block_size - 1) // block_size
    cache, nb = indexer_cache(device, g, batch * pools, block_size)
    perm = torch.randperm(nb, generator=g, device=device).to(torch.int32)
    bt = perm[: batch * per_req].view(batch, per_req).contiguous()
    qf = torch.randn(batch, 1, heads, INDEX_DIM, generator=g, device=device)
    q = (qf * (448.0 / qf.abs().amax(dim=-1, keepdim=True))).to(torch.float8_e4m3fn)
    w = torch.randn(batch, heads, generator=g, device=device) * heads ** -0.5
    lens = torch.full((batch,), pools, dtype=torch.int32, device=device)
    lens[1:] -= torch.randint(0, max(1, min(4096, pools // 2)), (batch - 1,), generator=g, device=device,
                              dtype=torch.int32)
    return q, cache, w.contiguous(), lens, bt, pools


def indexer_prefill_inputs(device, g, rows=2048, context=262144, block_size=64, heads=INDEX_HEADS):
    """Prefill indexer scoring at the full context (the reference's TP4
    prefill indexer benchmark, docs/BENCHMARKS.md:27-34): one request whose
    last `rows` tokens (positions context - rows .. context - 1) each score
    the complete pools before them, 65536 pools of 4 tokens in 1024 pages of
    64 placed at random.  Returns (q fp8 [rows, 1, H, 128], cache, weights
    fp32 [rows, H], context_lens int32 [rows] = (position + 1) // 4,
    block_table int32 [rows, 1024] (the request's table as a stride-0 view:
    every row reads the same table), max_model_len (pools))."""
    pools = context // INDEX_KPOOL
    per_req = (pools + block_size - 1) // block_size
    cache, nb = indexer_cache(device, g, pools, block_size)
    table = torch.randperm(nb, generator=g, device=device).to(torch.int32)[:per_req]
    bt = table[None, :].expand(rows, per_req)   # one table, shared by every row (row stride 0)
    qf = torch.randn(rows, 1, heads, INDEX_DIM, generator=g, device=device)
    q = (qf * (448.0 / qf.abs().amax(dim=-1, keepdim=True))).to(torch.float8_e4m3fn)
    w = torch.randn(rows, heads, generator=g, device=device) * heads ** -0.5
    pos = context - rows + torch.arange(rows, device=device)
    lens = ((pos + 1) // INDEX_KPOOL).to(torch.int32)
    return q, cache, w.contiguous(), lens, bt, pools


def indexer_bytes(lens: torch.Tensor, heads=INDEX_HEADS) -> int:
    """Algorithmic bytes of the logits: each valid pool key (128 fp8 bytes +
    4-byte scale) once per query, q and weights in, fp32 logits out."""
    n = int(lens.clamp(min=0).sum().item())
    t = lens.numel()
    return n * (INDEX_DIM + 4) + t * heads * (INDEX_DIM + 4) + n * 4


def indexer_flops(lens: torch.Tensor, heads=INDEX_HEADS) -> int:
    """FP8 multiply-adds of the logits as FLOPs: 2 * 128 per (valid pool
    key, head) of each query row."""
    return 2 * INDEX_DIM * heads * int(lens.clamp(min=0).sum().item())


# ----------------------------------------------------------------- bytes

def writer_bytes(n_rows: int) -> int:
    """Algorithmic bytes of store_int8: bf16 row in, int64 slot in, 528-B row out."""
    return n_rows * (LATENT * 2 + 8 + ROW_BYTES)


def mla_bytes(idx: torch.Tensor, n_rows: int, heads: int = HEADS) -> int:
    """Gathered valid rows + indices + q + out (split partials not counted)."""
    t = idx.shape[0]
    valid = int(((idx >= 0) & (idx < n_rows)).sum().item())
    return valid * ROW_BYTES + t * (idx.shape[-1] * 4 + 2 * heads * LATENT * 2)


def mla_flops(idx: torch.Tensor, n_rows: int, heads: int = HEADS) -> int:
    valid = int(((idx >= 0) & (idx < n_rows)).sum().item())
    return 4 * heads * LATENT * valid


def human(n: float) -> str:
    return f"{n:.3g}"


__all__ = [n for n in dir() if not n.startswith("_") and n not in ("math", "torch", "annotations")]
