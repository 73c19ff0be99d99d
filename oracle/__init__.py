"""CPU oracle for the GLM-5.3 decode hot path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
CPU-baseline leg of bench.py, always as the checker.  The product modules
(titan_kv, titan_mla, titan_moe_align) never import it.

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
    return len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)


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

