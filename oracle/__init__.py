"""CPU oracle for the GLM-5.3 decode hot path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
CPU-baseline leg of bench.py, always as the reference results are compared
against (never as the thing measured or shipped).  The product modules
(titan_kv, titan_mla, titan_moe_align, titan_moe_w4a16, sparse_utils,
sparse_indexer) never import it.

The arithmetic lives in glm53_oracle.c (built by oracle/Makefile into
liboracle.so); this module wraps it for numpy arrays and restates the two
pieces of reference host logic the tests need:

* choose_num_kv_splits  -- kernels/titan_mla.py:432-449
* moe_patterns          -- benchmarks/moe_align.py:49-55

and, in numpy, the request-relative index conversion the reference's adapter
runs before the attention (integration/titan_backend.py:48-52, vLLM's
triton_convert_req_index_to_global_index, not available here):

* convert_req_index     -- parity with vLLM unpinned; pinned by invariants
  (identity table, page/offset decomposition, masking) and by attention over
  the logically gathered cache (tests/test_oracle.py).
* expand_pools          -- the indexer's kpool expansion, following the
  reference's CPU model (tests/verify_indexer_sharding.py:72-79); pinned by
  an independent set formulation and closed-form cases (tests/test_oracle.py).

Pinning (what each function is checked against, in tests/test_oracle.py):
* store_int8: exact rational arithmetic (fractions.Fraction) on golden rows,
  closed-form special cases (zero row, amax element -> +-127, tail bytes,
  negative slot), brute force over small rows.
* moe_align: the reference's published postpad known answers
  (docs/measurements.json), an independent pairwise formulation, a numpy
  argsort formulation, and the 856-case sweep of benchmarks/moe_align.py:58-67.
* sparse_mla: textbook float64 attention (oracle_sparse_mla_f64 and a numpy
  restatement), invariants (split-count invariance, all-masked -> 0, masking
  of positive out-of-range indices, permutation invariance, one valid row,
  q = 0 gives the mean row).
* moe_w4a16 (+ unpack_w4 / pack_w4 / repack_w4a16), the expert GEMMs after
  the aligner (vLLM's fused Marlin MoE at integration/patch_moe_align.py:
  17-44, composed as profiles/sm74/titan_prefill/marlin.py:424-444): bit
  brute force of the packing and of the tile order, closed forms from
  uniform weights and from single codes per expert (every index of the
  layer), the SiLU clamp, route invariants and an independent torch
  formulation (tests/test_oracle_moe_w4a16.py).  The clamp's exact form
  (gate clamped above, up clamped both ways, limit 10) is vLLM's and is not
  in the reference: parity of that detail with vLLM is unpinned.
* e4m3_to_f32 / fp8_paged_mqa_logits, the indexer's decode scoring (vLLM's
  fp8_paged_mqa_logits_triton, called at integration/patch_decode_indexer.py:
  34-44, computing DeepGEMM's published definition): torch's float8_e4m3fn
  decoding of all 256 codes, the closed form of a unit query, paging
  invariance and masking, and an independent torch formulation
  (tests/test_oracle_indexer.py).  Parity with vLLM's kernel itself is
  unpinned (not in the container).
* order_key / indexer_topk, the top-k per row whose output is pool_topk
  (consumed at integration/patch_indexer_sharding.py:58-79): brute-force
  selection on normal, tied, short and special-value rows
  (tests/test_oracle_indexer.py).  The order inside ties (smaller position
  first, NaN below -inf) is this library's definition (vLLM's tie order is
  not part of the reference).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
LOG2E = 1.4426950408889634
ROW_BYTES = 528
LATENT = 512

_lib = None


def build(force: bool = False) -> Path:
    """Compile liboracle.so with the committed Makefile."""
    src = HERE / "glm53_oracle.c"
    if force or not LIB_PATH.exists() or LIB_PATH.stat().st_mtime < src.stat().st_mtime:
        subprocess.run(["make", "-s", "-C", str(HERE)] + (["-B"] if force else []), check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        P, I64, I, F, D = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_double
        L.oracle_store_int8.argtypes = [P, I64, P, I64, I64, I64, P, I64, I]
        L.oracle_store_int8.restype = None
        L.oracle_quantize_row.argtypes = [P, P]
        L.oracle_moe_align.argtypes = [P, I64, P, P, P]
        L.oracle_moe_align_pairwise.argtypes = [P, I64, P, P, P]
        L.oracle_moe_align_repeat.argtypes = [P, I64, P, P, P, I64]
        L.oracle_sparse_mla.argtypes = [P, I64, I64, P, I64, I64, P, I64, I64, I64, I64, F, I64, I64, I64, F, P, I64, I64, I]
        L.oracle_sparse_mla.restype = None
        L.oracle_sparse_mla_f64.argtypes = [P, I64, I64, P, I64, I64, P, I64, I64, I64, I64, D, P, I]
        L.oracle_sparse_mla_f64.restype = None
        L.oracle_abi_version.restype = I
        assert L.oracle_abi_version() == 3
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


# --------------------------------------------------------------------------
# bf16 helpers (round to nearest even, as torch / Triton convert)
# --------------------------------------------------------------------------

def bf16_to_f32(u16: np.ndarray) -> np.ndarray:
    return (np.asarray(u16, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


# --------------------------------------------------------------------------
# store_int8 (kernels/titan_kv.py:7-28)
# --------------------------------------------------------------------------

def store_int8(x_u16: np.ndarray, cache: np.ndarray, slots: np.ndarray, nthreads: int = 1) -> None:
    """Write rows of x (bf16 bits, [N, >=512], last dim contiguous) into the
    uint8 cache [nb, block, >=528] (modified in place) at the given slots."""
    assert x_u16.dtype == np.uint16 and x_u16.ndim == 2 and x_u16.strides[1] == 2
    assert cache.dtype == np.uint8 and cache.ndim == 3 and cache.strides[2] == 1
    slots = np.ascontiguousarray(np.asarray(slots).reshape(-1), dtype=np.int64)
    assert slots.size <= x_u16.shape[0]
    lib().oracle_store_int8(_ptr(x_u16), x_u16.strides[0] // 2, _ptr(cache), cache.strides[0],
                            cache.strides[1], cache.shape[1], _ptr(slots), slots.size, nthreads)


def quantize_rows(x_u16: np.ndarray, nthreads: int = 1) -> np.ndarray:
    """Return the [N, 528] uint8 rows for bf16 latents [N, 512]."""
    x_u16 = np.ascontiguousarray(x_u16, dtype=np.uint16)
    n = x_u16.shape[0]
    cache = np.zeros((n, 1, ROW_BYTES), dtype=np.uint8)
    store_int8(x_u16, cache, np.arange(n, dtype=np.int64), nthreads)
    return cache.reshape(n, ROW_BYTES)


def row_scales(rows: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(rows[:, LATENT:LATENT + 4]).view(np.float32).reshape(-1)


def dequantize(rows: np.ndarray) -> np.ndarray:
    """float64 [N, 512] = int8 values x fp32 scale."""
    q = rows[:, :LATENT].view(np.int8).astype(np.float64)
    return q * row_scales(rows).astype(np.float64)[:, None]


# --------------------------------------------------------------------------
# MoE align (benchmarks/moe_align.py:23-67)
# --------------------------------------------------------------------------

def moe_align(ids, pairwise: bool = False):
    flat = np.ascontiguousarray(np.asarray(ids).reshape(-1), dtype=np.int64)
    R = flat.size
    sorted_ids = np.empty(R * 8, dtype=np.int32)
    experts = np.empty(R, dtype=np.int32)
    postpad = np.empty(1, dtype=np.int32)
    fn = lib().oracle_moe_align_pairwise if pairwise else lib().oracle_moe_align
    fn(_ptr(flat), R, _ptr(sorted_ids), _ptr(experts), _ptr(postpad))
    return sorted_ids, experts, postpad


def moe_align_repeat(ids, iters: int) -> None:
    """oracle_moe_align `iters` times over the same routes (the CPU
    baseline's timing loop; outputs discarded)."""
    flat = np.ascontiguousarray(np.asarray(ids).reshape(-1), dtype=np.int64)
    R = flat.size
    sorted_ids = np.empty(R * 8, dtype=np.int32)
    experts = np.empty(R, dtype=np.int32)
    postpad = np.empty(1, dtype=np.int32)
    lib().oracle_moe_align_repeat(_ptr(flat), R, _ptr(sorted_ids), _ptr(experts), _ptr(postpad), int(iters))


def moe_patterns(batch: int, rng) -> dict:
    """The seven routing patterns of benchmarks/moe_align.py:49-55 (rng is a
    random.Random; only random_top8 consumes it)."""
    routes = batch * 8
    return {"distinct": list(range(routes)), "shared_top8": list(range(8)) * batch,
            "random_top8": [e for _ in range(batch) for e in rng.sample(range(288), 8)],
            "all_one_expert": [173] * routes, "seven_experts": [i % 7 for i in range(routes)],
            "invalid_mixed": [-1 if i % 5 == 0 else 288 if i % 7 == 0 else i % 11 for i in range(routes)],
            "all_invalid": [-1] * routes}


# --------------------------------------------------------------------------
# Sparse MLA (kernels/titan_mla.py)
# --------------------------------------------------------------------------

def choose_num_kv_splits(num_tokens: int, num_head_groups: int, index_topk: int, sm_count: int) -> int:
    """Restatement of kernels/titan_mla.py:432-449."""
    baseline = num_tokens * num_head_groups
    if baseline == 0 or baseline * 4 >= sm_count:
        return 1
    ideal = 1 << max(0, (max(1, index_topk // 128) - 1).bit_length())
    max_splits = max(1, sm_count // baseline)
    max_splits = 1 << (max_splits.bit_length() - 1)
    n = min(ideal, max_splits)
    while n > 1 and index_topk % n != 0:
        n //= 2
    return max(1, n)


def _mla_args(q_u16, rows, idx):
    assert q_u16.dtype == np.uint16 and q_u16.ndim == 3 and q_u16.strides[2] == 2
    assert rows.dtype == np.uint8 and rows.ndim == 2 and rows.strides[1] == 1 and rows.shape[1] >= ROW_BYTES
    idx = np.asarray(idx, dtype=np.int32)
    if idx.ndim == 3:
        idx = idx[:, 0, :]
    idx = np.ascontiguousarray(idx)
    return q_u16, rows, idx


def sparse_mla(q_u16: np.ndarray, rows: np.ndarray, idx: np.ndarray, sm_scale: float,
               n_splits: int = 1, block_n: int = 32, nthreads: int = 1, groups: int = 1,
               lazy: float = 0.0) -> np.ndarray:
    """Faithful restatement: returns bf16 bits [T, H, 512].  groups > 1 deals
    each split's tiles round-robin to that many online-softmax streams merged
    by a pairwise tree; lazy > 0 moves a stream's max only when a tile exceeds
    it by more than `lazy`.  groups = 1, lazy = 0 is the reference."""
    q_u16, rows, idx = _mla_args(q_u16, rows, idx)
    T, H, _ = q_u16.shape
    topk = idx.shape[1]
    out = np.zeros((T, H, LATENT), dtype=np.uint16)
    sm_scale_log2 = np.float32(sm_scale * LOG2E)
    lib().oracle_sparse_mla(_ptr(q_u16), q_u16.strides[0] // 2, q_u16.strides[1] // 2, _ptr(rows),
                            rows.strides[0], rows.shape[0], _ptr(idx), idx.strides[0] // 4, T, H, topk,
                            float(sm_scale_log2), int(n_splits), int(block_n), int(groups), float(lazy),
                            _ptr(out),
                            out.strides[0] // 2, out.strides[1] // 2, nthreads)
    return out


def sparse_mla_f64(q_u16: np.ndarray, rows: np.ndarray, idx: np.ndarray, sm_scale: float,
                   nthreads: int = 1) -> np.ndarray:
    """Textbook float64 attention over the dequantised rows: [T, H, 512]."""
    q_u16, rows, idx = _mla_args(q_u16, rows, idx)
    T, H, _ = q_u16.shape
    out = np.zeros((T, H, LATENT), dtype=np.float64)
    lib().oracle_sparse_mla_f64(_ptr(q_u16), q_u16.strides[0] // 2, q_u16.strides[1] // 2, _ptr(rows),
                                rows.strides[0], rows.shape[0], _ptr(idx), idx.strides[0] // 4, T, H,
                                idx.shape[1], float(sm_scale), _ptr(out), nthreads)
    return out


def default_threads() -> int:
    """Host threads for the oracle: the CPUs this process may run on, at
    most 16 (the host CPU share of one GPU on an 8-GPU node)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    return max(1, min(16, n))


def convert_req_index(req_id: np.ndarray, block_table: np.ndarray, indices: np.ndarray,
                      block_size: int, page_rows: int | None = None) -> np.ndarray:
    """Request-relative token positions -> flat cache rows (int32).

    For token t (request r = req_id[t]) and position p = indices[t, k]:
    -1 if p < 0, r is not a block-table row, or p // block_size >= max_blocks;
    otherwise block_table[r, p // block_size] * page_rows + p % block_size in
    wrapping 32-bit arithmetic (page_rows defaults to block_size)."""
    page_rows = block_size if page_rows is None else page_rows
    req_id = np.asarray(req_id, dtype=np.int64)
    bt = np.asarray(block_table, dtype=np.int32)
    idx = np.asarray(indices, dtype=np.int64)
    num_reqs, max_blocks = bt.shape
    out = np.full(idx.shape, -1, dtype=np.int32)
    for t in range(idx.shape[0]):
        r = req_id[t]
        if r < 0 or r >= num_reqs:
            continue
        p = idx[t]
        blk = np.where(p >= 0, p // block_size, max_blocks)
        ok = (p >= 0) & (blk < max_blocks)
        base = bt[r, np.where(ok, blk, 0)].astype(np.uint32) if max_blocks else np.zeros(p.shape, np.uint32)
        row = base * np.uint32(page_rows) + (p - np.maximum(blk, 0) * block_size).astype(np.uint32)
        out[t] = np.where(ok, row.astype(np.uint32).view(np.int32), -1)
    return out


def expand_pools(pool_ids: np.ndarray, seq_lens, pool_size: int, out_cols: int | None = None) -> np.ndarray:
    """Pool ids [rows, K] -> token positions (tests/verify_indexer_sharding.py:
    72-79): slot j * pool_size + o holds pool_ids[r, j] * pool_size + o (-1 for
    a negative id); with seq_lens, the next pool_size - 1 slots hold the tail
    tokens seq_lens[r] // pool_size * pool_size + o for o < seq_lens[r] %
    pool_size (-1 otherwise).  Slots up to out_cols past that are -1."""
    p = np.asarray(pool_ids, dtype=np.int64)
    rows, k = p.shape
    width = k * pool_size + (pool_size - 1 if seq_lens is not None else 0)
    out_cols = width if out_cols is None else out_cols
    out = np.full((rows, out_cols), -1, dtype=np.int64)
    offs = np.arange(pool_size)
    body = np.where(p[:, :, None] >= 0, p[:, :, None] * pool_size + offs[None, None, :], -1).reshape(rows, -1)
    n = min(out_cols, k * pool_size)
    out[:, :n] = body[:, :n]
    if seq_lens is not None:
        s = np.asarray(seq_lens, dtype=np.int64)
        tail = np.where(offs[None, : pool_size - 1] < (s % pool_size)[:, None],
                        (s // pool_size * pool_size)[:, None] + offs[None, : pool_size - 1], -1)
        lo, hi = k * pool_size, min(out_cols, width)
        if hi > lo:
            out[:, lo:hi] = tail[:, : hi - lo]
    return out.astype(np.int32)



# --------------------------------------------------------------------------
# W4A16 group-32 MoE expert GEMMs (the consumer of moe_align; vLLM's fused
# Marlin MoE at integration/patch_moe_align.py:17-44, composed as in
# profiles/sm74/titan_prefill/marlin.py:424-444)
# --------------------------------------------------------------------------

def unpack_w4(words: np.ndarray) -> np.ndarray:
    """int32 [..., K/8] GPTQ-packed words -> uint8 codes [..., K]: code k of
    a row is bits 4*(k % 8) .. +3 of word k // 8."""
    w = np.ascontiguousarray(words).view(np.uint32)
    shifts = 4 * np.arange(8, dtype=np.uint32)
    return ((w[..., None] >> shifts) & 0xF).astype(np.uint8).reshape(*w.shape[:-1], 8 * w.shape[-1])


def pack_w4(codes: np.ndarray) -> np.ndarray:
    """Inverse of unpack_w4: uint8 codes [..., K] (values 0..15) -> int32 [..., K/8]."""
    c = np.asarray(codes, dtype=np.uint32).reshape(*codes.shape[:-1], codes.shape[-1] // 8, 8)
    return (c << (4 * np.arange(8, dtype=np.uint32))).sum(axis=-1, dtype=np.uint32).view(np.int32)


def repack_w4a16(words: np.ndarray) -> np.ndarray:
    """The kernels' tile order (glm53_moe_w4a16_repack): [E, n_out, K/8] ->
    int32 [E, n_out/16, K/128, 64, 4].  Lane l of tile (e, nt, c) holds row
    16*nt + l%16; its word i holds codes k = 32*(4c+i) + 8*(l//16) + 2j in
    bits 4j and k + 1 in bits 16 + 4j (j = 0..3)."""
    codes = unpack_w4(words)                         # [E, n, K]
    E, n, K = codes.shape
    c = codes.reshape(E, n // 16, 16, K // 128, 4, 4, 8)   # e, nt, row, chunk, i, q, kk
    c = c.transpose(0, 1, 3, 5, 2, 4, 6).astype(np.uint32)  # e, nt, chunk, q, row, i, kk
    shift = np.array([0, 16, 4, 20, 8, 24, 12, 28], dtype=np.uint32)
    w = (c << shift).sum(axis=-1, dtype=np.uint32)          # e, nt, chunk, q, row, i
    return w.reshape(E, n // 16, K // 128, 64, 4).view(np.int32)


def repack_w4a16_scales(scales: np.ndarray) -> np.ndarray:
    """The scales' tile order (glm53_moe_w4a16_repack): [E, n_out, K/32] ->
    [E, n_out/16, K/128, 16, 4]; element [e, nt, c, r, g] is the scale of row
    16*nt + r, group 4c + g."""
    E, n, G = scales.shape
    return np.ascontiguousarray(scales.reshape(E, n // 16, 16, G // 4, 4).transpose(0, 1, 3, 2, 4))


def _dequant(words: np.ndarray, scales_u16: np.ndarray) -> np.ndarray:
    """(q - 8) * s in float64 (exact), [n_out, K]."""
    q = unpack_w4(words).astype(np.float64) - 8.0
    s = bf16_to_f32(scales_u16).astype(np.float64)
    return q * np.repeat(s, 32, axis=-1)


def moe_w4a16(x_u16: np.ndarray, w13: np.ndarray, s13: np.ndarray, w2: np.ndarray, s2: np.ndarray,
              topk_weights: np.ndarray, topk_ids: np.ndarray, clamp_limit: float | None = 10.0,
              cache: dict | None = None):
    """The MoE layer for tokens x (bf16 bits [T, K]) and routes (topk_ids,
    topk_weights [T, topk]); weights in checkpoint packing (w13 int32 [E, 2N,
    K/8], s13 bf16 bits [E, 2N, K/32], w2 [E, K, N/8], s2 [E, K, N/32]).

    Rounding points (those of the fused Marlin MoE: bf16 intermediate
    buffers, moe_sum over fp32): c1 = bf16(x . W13^T) with an exact float64
    dot, c2 = bf16(silu(min(g, L)) * clip(u, -L, L)) computed in fp32,
    c3 = bf16(fp32(w) * fp32(c2 . W2^T)), out = bf16 of the fp32 sum of the
    token's c3 in slot order.  A route whose expert is outside [0, E) gives
    c3 = 0.  Returns (out bf16 bits [T, K], c2 bf16 bits [T*topk, N] with
    zero rows for dropped routes).  `cache` (a dict, optional) keeps the
    dequantised experts between calls on the same weights."""
    cache = {} if cache is None else cache
    c1 = moe_w4a16_c1(x_u16, w13, s13, w2, s2, topk_ids, cache)
    act = f32_to_bf16(moe_activation(c1, clamp_limit))
    routed = ((np.asarray(topk_ids) >= 0) & (np.asarray(topk_ids) < w13.shape[0])).reshape(-1)
    act[~routed] = 0
    out, _ = moe_w4a16_down(act, w13, s13, w2, s2, topk_weights, topk_ids, cache)
    return out, act


def moe_w4a16_c1(x_u16: np.ndarray, w13: np.ndarray, s13: np.ndarray, w2: np.ndarray, s2: np.ndarray,
                 topk_ids: np.ndarray, cache: dict | None = None, with_magnitude: bool = False):
    """c1 = bf16(x . W13^T) (exact float64 dot) of every route as float32
    [T*topk, 2N] (gate then up), row t * topk + j; zero rows for routes whose
    expert is outside [0, E).  with_magnitude: also return, per output,
    280 * sum_k |s_k x_k| (s_k the group scale of feature k): the size of
    the partial sums an fp32 evaluation on biased codes passes through
    ((128 + q) codes and a -136 seed: |128 + q| + 136 <= 280), which scales
    its rounding error when the result itself is small."""
    x = bf16_to_f32(x_u16).astype(np.float64)
    E = w13.shape[0]
    T, topk = topk_ids.shape
    ids = np.asarray(topk_ids, dtype=np.int64)
    c1 = np.zeros((T * topk, w13.shape[1]), dtype=np.float32)
    mag = np.zeros_like(c1)
    cache = {} if cache is None else cache
    for t in range(T):
        for j in range(topk):
            e = int(ids[t, j])
            if 0 <= e < E:
                W13 = _experts(cache, e, w13, s13, w2, s2)[0].astype(np.float64)
                c1[t * topk + j] = bf16_to_f32(f32_to_bf16((W13 @ x[t]).astype(np.float32)))
                if with_magnitude:
                    s = np.abs(bf16_to_f32(s13[e]).astype(np.float64))          # [2N, K/32]
                    xs = np.abs(x[t]).reshape(-1, 32).sum(axis=1)                # [K/32]
                    mag[t * topk + j] = 280.0 * (s @ xs)
    return (c1, mag) if with_magnitude else c1


def moe_activation(c1: np.ndarray, clamp_limit: float | None = 10.0) -> np.ndarray:
    """silu(min(g, L)) * clip(u, -L, L) in fp32 for c1 rows [..., 2N] (gate
    then up); returns fp32 [..., N] before the bf16 rounding."""
    L = np.float32(np.inf if clamp_limit is None else clamp_limit)
    N = c1.shape[-1] // 2
    g = np.minimum(c1[..., :N].astype(np.float32), L)
    u = np.clip(c1[..., N:].astype(np.float32), -L, L)
    with np.errstate(over="ignore"):
        return (g / (np.float32(1) + np.exp(-g)) * u).astype(np.float32)


def _experts(cache: dict, e: int, w13, s13, w2, s2):
    """Expert e's dequantised (W13, W2) in fp32, kept in `cache`; (q - 8) * s
    is exact in fp32 (a 4-bit code times a bf16 scale)."""
    if e not in cache:
        cache[e] = (_dequant(w13[e], s13[e]).astype(np.float32), _dequant(w2[e], s2[e]).astype(np.float32))
    return cache[e]


def moe_w4a16_down(act_u16: np.ndarray, w13: np.ndarray, s13: np.ndarray, w2: np.ndarray, s2: np.ndarray,
                   topk_weights: np.ndarray, topk_ids: np.ndarray, cache: dict | None = None):
    """The layer's second half on given activations c2 (bf16 bits [T*topk, N],
    row t * topk + j): c3 = bf16(fp32(w) * fp32(c2 . W2^T)) with an exact
    float64 dot, out = bf16 of the fp32 sum of the token's c3 in slot order;
    a route whose expert is outside [0, E) gives c3 = 0.  Returns (out bf16
    bits [T, K], c3 float32 [T, topk, K])."""
    E = w2.shape[0]
    K = w2.shape[1]
    T, topk = topk_ids.shape
    ids = np.asarray(topk_ids, dtype=np.int64)
    tw = np.asarray(topk_weights, dtype=np.float32)
    c3 = np.zeros((T, topk, K), dtype=np.float32)
    cache = {} if cache is None else cache
    for t in range(T):
        for j in range(topk):
            e = int(ids[t, j])
            if not 0 <= e < E:
                continue
            W2 = _experts(cache, e, w13, s13, w2, s2)[1].astype(np.float64)
            y = (W2 @ bf16_to_f32(act_u16[t * topk + j]).astype(np.float64)).astype(np.float32)
            c3[t, j] = bf16_to_f32(f32_to_bf16(tw[t, j] * y))
    out = np.zeros((T, K), dtype=np.float32)
    for j in range(topk):
        out += c3[:, j]
    return f32_to_bf16(out), c3


# --------------------------------------------------------------------------
# Sparse indexer decode scoring: FP8 paged MQA logits (DeepGEMM's published
# fp8_paged_mqa_logits semantics; vLLM's fp8_paged_mqa_logits_triton as the
# reference calls it, integration/patch_decode_indexer.py:34-44) and the
# top-k pool selection (integration/patch_decode_indexer.py:64-72)
# --------------------------------------------------------------------------

def e4m3_to_f32(codes: np.ndarray) -> np.ndarray:
    """OCP FP8 E4M3 (e4m3fn) bytes -> float32: bias 7, subnormals m * 2^-9,
    0x7F / 0xFF NaN, no infinities."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 0x7
    mag = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    out = sign * mag
    out = np.where((c & 0x7F) == 0x7F, np.nan, out)
    return out.astype(np.float32)


def fp8_paged_mqa_logits(q_u8: np.ndarray, pages: np.ndarray, block_size: int, weights: np.ndarray,
                         context_lens: np.ndarray, block_table: np.ndarray, max_len: int,
                         clean: bool = True, bound: bool = False):
    """q_u8 uint8 [T, H, 128]; pages uint8 [num_blocks, page_bytes] (block_size
    x 128 key bytes, then block_size float32 scales); weights [T, H]; per-row
    context_lens [T] and block_table [T, max_blocks].  Returns float64 logits
    [T, max_len] (NaN where not written: positions >= context when not clean);
    with bound=True also the float64 sum over heads and dims of
    |w s q k| (the magnitude an fp32 accumulation error scales with)."""
    T, H, D = q_u8.shape
    nb = pages.shape[0]
    table = e4m3_to_f32(np.arange(256, dtype=np.uint8)).astype(np.float64)
    out = np.full((T, max_len), np.nan)
    mag = np.zeros((T, max_len))
    cap = block_table.shape[1] * block_size
    for t in range(T):
        n = int(min(max(int(context_lens[t]), 0), cap))
        if clean:
            out[t, n:] = -np.inf
        n = min(n, max_len)
        j = np.arange(n)
        blk = np.asarray(block_table[t, j // block_size], dtype=np.int64)
        ok = (blk >= 0) & (blk < nb)
        off = j % block_size
        b = np.where(ok, blk, 0)
        kbytes = pages[b[:, None], off[:, None] * D + np.arange(D)[None, :]]          # [n, D]
        sbytes = pages[b[:, None], block_size * D + 4 * off[:, None] + np.arange(4)[None, :]]
        s = np.ascontiguousarray(sbytes).view(np.float32).reshape(n).astype(np.float64)
        k = table[kbytes]
        q = table[q_u8[t]]                                                             # [H, D]
        w = np.asarray(weights[t], dtype=np.float64)
        dots = k @ q.T                                                                 # [n, H]
        # relu as fmax: a (key, head) product that is NaN (an E4M3 NaN code in
        # k or q) contributes 0, as the kernels' fmaxf(x, 0) gives
        val = (np.fmax(s[:, None] * dots, 0.0) * w[None, :]).sum(axis=1)
        out[t, :n] = np.where(ok, val, -np.inf)
        if bound:
            kk = np.nan_to_num(np.abs(k), nan=0.0)
            qq = np.nan_to_num(np.abs(q), nan=0.0)
            terms = np.abs(s)[:, None] * (kk @ qq.T) * np.abs(w)[None, :]
            terms = np.where(np.isnan(s[:, None] * dots), 0.0, terms)                 # dropped terms: exactly 0
            mag[t, :n] = np.where(ok, terms.sum(axis=1), 0.0)
    return (out, mag) if bound else out


def order_key(f: np.ndarray) -> np.ndarray:
    """Order-preserving uint32 key of float32 values (larger float -> larger
    key; NaN -> 0, below everything)."""
    u = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32)
    key = np.where(u & 0x80000000, ~u, u | 0x80000000).astype(np.uint32)
    return np.where(np.isnan(np.asarray(f, dtype=np.float32)), np.uint32(0), key)


def indexer_topk(logits: np.ndarray, lengths: np.ndarray, k: int) -> np.ndarray:
    """For each row, the positions of the k largest logits among [0, len)
    (NaN lowest, ties by smaller position), ascending; -1 padding."""
    rows = logits.shape[0]
    out = np.full((rows, k), -1, dtype=np.int32)
    for r in range(rows):
        n = int(min(max(int(lengths[r]), 0), logits.shape[1]))
        keys = order_key(logits[r, :n].astype(np.float32)).astype(np.int64)
        idx = np.arange(n)
        order = np.lexsort((idx, -keys))[:k]     # key descending, position ascending
        sel = np.sort(order)
        out[r, :sel.size] = sel
    return out
